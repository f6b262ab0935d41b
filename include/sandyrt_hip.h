/*
 * sandyrt_hip.h -- C ABI of the MI355X (gfx950) backend for SandyRT's
 * data-parallel hot path.
 *
 * The reference dispatches every KernelIR op through one C++ launcher per
 * kernel family, `launch_cuda_<family>(const CudaLaunchContext&, const
 * Cuda<Family>Program&)` (src/device/cuda/CudaKernels.h:109-159), selected
 * by `CudaDevice::run` (src/device/cuda/CudaDevice.cpp:520-578).  Each entry
 * point below replaces one of those launchers.  Instead of the C++ context it
 * takes plain tensor descriptors (device pointer, dtype, dims, strides,
 * storage offset -- the fields of CudaDeviceBufferView/TensorViewDesc,
 * src/device/cuda/CudaKernels.h:19-28, src/device/DeviceTypes.h:25-29), the
 * op attributes that the Cuda<Family>Program carries, and a hipStream_t.
 *
 * Conventions
 *   - Every call is stream-ordered on `stream` (a hipStream_t, NULL = the
 *     default stream) and returns without synchronising the host.
 *   - Return value 0 = success.  Non-zero = failure; a message worded like
 *     the reference's Result<> error is written to err[0..err_cap).
 *   - dtype codes follow sandy::core::DType (src/core/Tensor.h:13).
 *   - Float tensors are F32 or BF16 (bf16 stores round to nearest even,
 *     src/core/Tensor.h:43-49); index tensors are I32 or I64.
 *   - Value checks that depend on device data (expert ids, token ids,
 *     positions) cannot fail the call without a host round trip; kernels
 *     record them in a sticky per-device error word instead, read with
 *     sandy_hip_take_device_errors().
 */
#ifndef SANDYRT_HIP_H
#define SANDYRT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SANDY_HIP_MAX_RANK 8
#define SANDY_HIP_MAX_INPUTS 8
#define SANDY_HIP_MAX_SCALARS 32

enum SandyDType { SANDY_F32 = 0, SANDY_F16 = 1, SANDY_BF16 = 2, SANDY_I32 = 3, SANDY_I64 = 4, SANDY_U8 = 5 };

enum SandyStatus {
    SANDY_OK = 0,
    SANDY_ERR_INVALID = 1,     /* shape / dtype / attribute rejected */
    SANDY_ERR_UNSUPPORTED = 2, /* valid op this backend does not implement */
    SANDY_ERR_HIP = 3,         /* HIP runtime failure */
    SANDY_ERR_COMPILE = 4      /* hipRTC compilation failure */
};

/* Device-side value errors (bit flags of the sticky error word). */
enum SandyDeviceError {
    SANDY_DEVERR_EXPERT_ID = 1u << 0,   /* moe_gather topk expert id out of range */
    SANDY_DEVERR_TOKEN_ID = 1u << 1,    /* moe_scatter_sum token id out of range */
    SANDY_DEVERR_POSITION = 1u << 2,    /* rope position_ids must be non-negative */
    SANDY_DEVERR_GATHER_ID = 1u << 3,   /* embedding id out of range */
    SANDY_DEVERR_OFFSETS = 1u << 4,     /* moe_matmul invalid expert offsets */
    SANDY_DEVERR_BLOCK = 1u << 5,       /* paged block id outside the pool */
    SANDY_DEVERR_ATTN_POS = 1u << 6     /* attention position_offsets must be non-negative */
};

/* A strided view of device memory (TensorViewDesc, src/device/DeviceTypes.h:25-29). */
typedef struct SandyTensor {
    void* data;               /* device address of storage element 0 */
    int32_t dtype;            /* enum SandyDType */
    int32_t rank;             /* 0..8 */
    int64_t dims[SANDY_HIP_MAX_RANK];
    int64_t strides[SANDY_HIP_MAX_RANK]; /* in elements */
    int64_t storage_offset;              /* in elements */
} SandyTensor;

/*
 * A paged KV cache.  Every page holds `page_size` consecutive rows of the grow
 * dimension for all `prefix` leading elements: page = [prefix, page_size,
 * inner] (the reference's page layout, src/device/cuda/CudaPagedTensor.cpp:
 * 187-226, addressing src/device/cuda/CudaKernelUtils.cuh:82-108).  Pages live
 * in one pool allocation and are named by int32 block ids (pool + id *
 * page_stride elements) instead of the reference's per-page void* table.
 * page_stride 0 means dense pages (prefix * page_size * inner); a larger
 * stride lets K and V share one allocation with block b's K page and V page
 * side by side ([pages, 2, prefix, page_size, inner]: K at pool, V at pool +
 * prefix * page_size * inner, both with stride 2 * prefix * page_size * inner).
 */
typedef struct SandyPagedCache {
    void* pool;               /* device base address of the page pool (of page 0) */
    int32_t dtype;
    int32_t reserved;
    int64_t page_size;        /* rows of the grow dimension per page (power of two) */
    int64_t prefix;           /* elements before the grow dim, e.g. kv heads */
    int64_t inner;            /* elements after the grow dim, e.g. head dim */
    int64_t num_pages;        /* pool capacity in pages */
    int64_t page_stride;      /* elements from one page to the next; 0: prefix * page_size * inner */
} SandyPagedCache;

/*
 * The reference's own paged tensor, as CudaDevice hands it to a kernel
 * (CudaDeviceBufferView with paged = true, src/device/cuda/CudaKernels.h:
 * 19-28; pages built by CudaPagedTensorPool, CudaPagedTensor.cpp:187-226):
 * `pages` is the device array of page_count page start addresses (the
 * reference's void** page table), `dims` the logical shape -- [B, Hkv, T, D]
 * or [Hkv, T, D] with the grow dimension T at rank - 2 -- and a page holds
 * page_size rows of T for every leading element: [prefix, page_size, D] with
 * prefix = B * Hkv (rank 4) or Hkv.  One page list serves the whole batch,
 * so T is the batch's padded key length (addressing: CudaKernelUtils.cuh:
 * 82-108).
 */
typedef struct SandyPagedView {
    const void* pages;        /* device array of uint64 page addresses */
    int32_t dtype;
    int32_t rank;             /* 3 or 4 */
    int64_t dims[4];
    int64_t page_size;        /* power of two */
    int64_t page_count;       /* pages in the table (>= ceil(T / page_size)) */
} SandyPagedView;

/*
 * The reference's paged tensor in its general form, as an input of any
 * kernel family (CudaDeviceBufferView with paged = true, src/device/cuda/
 * CudaKernels.h:19-28, built by CudaDevice::run, CudaDevice.cpp:468-493):
 * `pages` is the device array of page_count page start addresses, `dims` the
 * logical shape, and page p holds rows [p * page_size, (p + 1) * page_size)
 * of dimension grow_dim for every leading element: [prefix, page_size, inner]
 * with prefix the product of the dims before grow_dim and inner the product
 * of those after it (addressing: CudaKernelUtils.cuh:82-108).  Elements on a
 * page the table lacks (ordinal >= page_count, or a null address) read as 0.
 */
typedef struct SandyPagedTensor {
    const void* pages;        /* device array of uint64 page addresses */
    int32_t dtype;            /* F32, BF16, I32 or I64 */
    int32_t rank;             /* 1..8 */
    int64_t dims[SANDY_HIP_MAX_RANK];
    int64_t grow_dim;         /* 0..rank-1 */
    int64_t page_size;        /* power of two */
    int64_t page_count;
} SandyPagedTensor;

#define SANDY_HIP_PAGED_STAGE_SLOTS 8

/* One node of a fused element-wise scalar DAG (ScalarNode, src/ir/KernelIR.h:346-355). */
typedef struct SandyScalarNode {
    uint32_t id;
    int32_t op;               /* sandy::ir::kernel_ir::ScalarOp order, KernelIR.h:317-337 */
    int32_t dtype;
    uint32_t input_index;     /* Load: which input */
    double constant;          /* Constant: the value */
    int32_t operand_count;    /* 0..2 */
    uint32_t operands[2];
} SandyScalarNode;

/* ---------------------------------------------------------------- library */

/* Version string of the backend ("sandyrt-hip <semver> gfx950"). */
const char* sandy_hip_version(void);

/* Reads and clears the sticky device error word of the current device after
 * synchronising `stream`.  *flags receives the SandyDeviceError bits; if any
 * bit is set the call returns SANDY_ERR_INVALID with the reference's message
 * for the lowest set bit.  Replaces the per-launch flag read-backs of
 * CudaRoPEKernels.cu:310-333, CudaGatherKernels.cu:291-294 and
 * CudaMoeScatterSumKernels.cu:218-239. */
int sandy_hip_take_device_errors(void* stream, uint32_t* flags, char* err, size_t err_cap);

/* ---------------------------------------------------------------- paged operands */

/*
 * Paged inputs of the families that read them (element-wise, norm, RoPE,
 * softmax, reduction, embedding gather, attention q and positions): the
 * reference reads such an input in place through load_float / load_int
 * (CudaKernelUtils.cuh:82-157); this backend gathers it into a dense
 * row-major copy, then the family's dense entry point reads the copy.  The
 * copy is exact, so the results are the same.
 *
 * sandy_hip_paged_to_dense: into dst, a contiguous tensor of src's shape and
 * dtype.  sandy_hip_paged_stage: into the library's per-device staging
 * buffer `slot` (0..SANDY_HIP_PAGED_STAGE_SLOTS-1, grow-only, allocated on
 * first use), described in *dense; it stays valid until the next stage call
 * of the same slot on that device, so one launch stages each of its paged
 * inputs in its own slot.  Calls that share a slot on one device and overlap
 * on different streams race.
 */
int sandy_hip_paged_to_dense(const SandyPagedTensor* src, const SandyTensor* dst, void* stream, char* err,
                             size_t err_cap);
int sandy_hip_paged_stage(const SandyPagedTensor* src, int32_t slot, SandyTensor* dense, void* stream, char* err,
                          size_t err_cap);

/* ---------------------------------------------------------------- fused groups */

/*
 * One fused element-wise group (ElementwiseKernelOp, src/ir/KernelIR.h:357-387;
 * replaces launch_cuda_elementwise, src/device/cuda/CudaElementwiseKernels.cu:
 * 189-213).  The scalar DAG is turned into straight-line gfx950 HIP C++ and
 * compiled with hipRTC on first use (cached by DAG hash).  broadcast[i] = 1
 * marks a right-aligned broadcast input (element index = linear % numel).
 */
int sandy_hip_elementwise(const SandyScalarNode* nodes, int32_t node_count, uint32_t result,
                          const SandyTensor* inputs, const int32_t* broadcast, int32_t input_count,
                          const SandyTensor* out, void* stream, char* err, size_t err_cap);

/*
 * NormKernelOp (src/ir/KernelIR.h:544-573; replaces launch_cuda_norm,
 * src/device/cuda/CudaNormKernels.cu:210-237).  kind 0 = RMSNorm
 * (weight may be NULL, bias must be NULL), kind 1 = LayerNorm (weight and
 * bias required).  Normalises the last dimension.
 */
int sandy_hip_norm(int32_t kind, const SandyTensor* x, const SandyTensor* weight,
                   const SandyTensor* bias, double epsilon, const SandyTensor* out,
                   void* stream, char* err, size_t err_cap);

/*
 * Residual add fused into the following RMSNorm -- the model pair
 * `x = __add(x, h); y = __rms_norm(x, w)` (src/models/tinyllama/
 * common.sandy.go:44-50) in one pass: sum_out = x + residual (rounded to the
 * output dtype, exactly the reference add), out = rms_norm(sum_out, weight).
 * sum_out may alias x.
 */
int sandy_hip_add_rms_norm(const SandyTensor* x, const SandyTensor* residual,
                           const SandyTensor* weight, double epsilon,
                           const SandyTensor* sum_out, const SandyTensor* out,
                           void* stream, char* err, size_t err_cap);

/*
 * RoPEKernelOp (src/ir/KernelIR.h:575-610; replaces launch_cuda_rope,
 * src/device/cuda/CudaRoPEKernels.cu:272-336).  position_ids may be NULL
 * (position = index along dim -2) or hold 1 (offset), seq or vector-count
 * entries.  rotary_dim < 0 means the full last dimension.  Negative position
 * ids set SANDY_DEVERR_POSITION instead of synchronising.
 */
int sandy_hip_rope(const SandyTensor* x, const SandyTensor* position_ids, double theta,
                   int64_t rotary_dim, int32_t split_half, const SandyTensor* out,
                   void* stream, char* err, size_t err_cap);
/* RoPE of two tensors that share position_ids, sequence length and head dim
 * (the q and k of one attention) in one launch: q_out / k_out are exactly
 * what two sandy_hip_rope calls produce.  Per-vector position ids (numel ==
 * vector count) fall back to one launch per tensor.  Fuses the program's two
 * RoPEKernelOps (src/models/tinyllama/common.sandy.go:24-25, lowered by
 * launch_cuda_rope, CudaKernels.h:109-159); the reference has no single
 * counterpart. */
int sandy_hip_rope_pair(const SandyTensor* q, const SandyTensor* k, const SandyTensor* position_ids, double theta,
                        int64_t rotary_dim, int32_t split_half, const SandyTensor* q_out, const SandyTensor* k_out,
                        void* stream, char* err, size_t err_cap);

/*
 * The cos/sin of a forward pass's RoPE positions, computed once and shared by
 * q, k and every layer.  No counterpart in the reference, which evaluates
 * powf/cosf/sinf per pair inside every RoPE launch (CudaRoPEKernels.cu:
 * 130-247); the values are those sandy_hip_rope uses (same angle, same
 * sin/cos).  cache [seq, rotary_dim / 2, 2] f32 = (cos, sin) of position(s) /
 * theta^(2i / d), d = dim (split_half) or rotary_dim; position_ids NULL
 * (position s), numel 1 (ids[0] + s) or numel seq (ids[s]).
 */
int sandy_hip_rope_cache(const SandyTensor* position_ids, int64_t seq, double theta, int64_t rotary_dim,
                         int64_t dim, int32_t split_half, const SandyTensor* cache, void* stream, char* err,
                         size_t err_cap);

/*
 * Split-half RoPE of q and k (k may be NULL) from a cache made by
 * sandy_hip_rope_cache for the same sequence length: bit-identical to
 * sandy_hip_rope_pair with that cache's positions, theta and rotary_dim.
 * Contiguous, 16-byte aligned rows whose half is 8, 16, ..., 256 elements.
 */
int sandy_hip_rope_pair_cached(const SandyTensor* q, const SandyTensor* k, const SandyTensor* cache,
                               const SandyTensor* q_out, const SandyTensor* k_out, void* stream, char* err,
                               size_t err_cap);

/* SoftmaxKernelOp (src/ir/KernelIR.h:494-515; replaces launch_cuda_softmax,
 * src/device/cuda/CudaSoftmaxKernels.cu:145-169).  Any axis. */
int sandy_hip_softmax(const SandyTensor* x, int64_t axis, const SandyTensor* out,
                      void* stream, char* err, size_t err_cap);

/* ReductionKernelOp with ReduceOp::Sum over one axis (replaces
 * launch_cuda_reduction, src/device/cuda/CudaKernels.cu:88-151). */
int sandy_hip_reduce_sum(const SandyTensor* x, int64_t axis, int32_t keep_dims,
                         const SandyTensor* out, void* stream, char* err, size_t err_cap);

/* GatherKernelOp / embedding (replaces launch_cuda_gather,
 * src/device/cuda/CudaGatherKernels.cu:97-117,360-387). */
int sandy_hip_gather(const SandyTensor* ids, const SandyTensor* table, const SandyTensor* out,
                     void* stream, char* err, size_t err_cap);

/* ---------------------------------------------------------------- attention */

/*
 * AttentionKernelOp on dense K/V (replaces launch_cuda_attention,
 * src/device/cuda/CudaAttentionKernels.cu:680-766).  q [B,Hq,Tq,D] (or rank
 * 3), k/v [B,Hkv,Tk,D]; position_offsets (NULL or [B]) shifts query
 * positions; window > 0 is a sliding window; scale <= 0 means 1/sqrt(D).
 */
int sandy_hip_attention(const SandyTensor* q, const SandyTensor* k, const SandyTensor* v,
                        const SandyTensor* position_offsets, int64_t window, double scale,
                        const SandyTensor* out, void* stream, char* err, size_t err_cap);

/*
 * Decode attention (Tq = 1) over a paged KV cache -- the reference's
 * AttentionKernelOp with paged K/V inputs (CudaAttentionKernels.cu:247-404,
 * 469-563).  q [B,Hq,1,D] bf16 or f32; k_cache/v_cache pages are [Hkv,
 * page_size, D]; block_table [B, max_blocks] int32 lists each sequence's pages
 * in order; position_offsets [B] (i32/i64) is the position of each query, so
 * keys 0..position (and >= position + 1 - window when window > 0) attend.
 * GQA head groups share one pass over their KV head (bf16: MFMA tiles).
 */
int sandy_hip_paged_attention(const SandyTensor* q, const SandyPagedCache* k_cache,
                              const SandyPagedCache* v_cache, const SandyTensor* block_table,
                              const SandyTensor* position_offsets, int64_t window, double scale,
                              const SandyTensor* out, void* stream, char* err, size_t err_cap);

/*
 * AttentionKernelOp with paged K/V exactly as the reference's engine passes
 * them (launch_cuda_attention with paged inputs, src/device/cuda/
 * CudaAttentionKernels.cu:680-766 over CudaPagedTensor pages; batched decode
 * is rank-4 attention with padded T and position_offsets,
 * src/core/TensorCalc.cpp:1167-1314).  q [B,Hq,Tq,D] (or rank 3) and out as
 * in sandy_hip_attention; k and v are reference-layout paged views.  Decode
 * (Tq = 1, bf16, D 64/128/256) runs the MFMA paged decode kernel reading the
 * page table directly; other shapes run the general attention kernel.
 * The decode kernel reads pages with 16-byte loads: a page address that is
 * null or not 16-byte aligned is recorded as SANDY_DEVERR_BLOCK and the page
 * contributes no keys.
 */
int sandy_hip_attention_paged_view(const SandyTensor* q, const SandyPagedView* k, const SandyPagedView* v,
                                   const SandyTensor* position_offsets, int64_t window, double scale,
                                   const SandyTensor* out, void* stream, char* err, size_t err_cap);

/*
 * sandy_hip_paged_attention without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops that forbid hipMalloc).  Same arguments,
 * semantics and errors as sandy_hip_paged_attention, restricted to the bf16
 * MFMA decode shapes (head dim 64/128/256, at most 16 q heads per kv head,
 * page_size a multiple of 16, 16-byte aligned q and pools); the split
 * partials, B * Hq * ceil(max_blocks * page_size / split) * (D + 2) floats,
 * must fit the library's fixed 8 MiB per-GPU scratch, else
 * SANDY_ERR_UNSUPPORTED.  Calls that overlap on one GPU share that scratch
 * and race.
 */
int sandy_hip_paged_attention_noalloc(const SandyTensor* q, const SandyPagedCache* k_cache,
                                      const SandyPagedCache* v_cache, const SandyTensor* block_table,
                                      const SandyTensor* position_offsets, int64_t window, double scale,
                                      const SandyTensor* out, void* stream, char* err, size_t err_cap);

/* ---------------------------------------------------------------- layout */

/* LayoutTransformKind, in the reference's order (src/ir/KernelIR.h:268-274). */
enum SandyLayoutKind {
    SANDY_LAYOUT_RESHAPE = 0,
    SANDY_LAYOUT_TRANSPOSE = 1,
    SANDY_LAYOUT_PERMUTE = 2,
    SANDY_LAYOUT_SLICE = 3,
    SANDY_LAYOUT_CONTIGUOUS = 4
};

/*
 * LayoutTransformKernelOp (replaces launch_cuda_layout_transform,
 * src/device/cuda/CudaLayoutTransformKernels.cu:25-78, dispatched at
 * CudaDevice.cpp:527-530): copies the logical elements of the strided view
 * `in` into `out` in row-major order -- the element count and dtype must
 * match, the shapes may differ (reshape).  The engine passes the input view
 * that a transpose or permute produced (Engine.cpp:606-754), so `kind` only
 * rejects SANDY_LAYOUT_SLICE, which is always an alias.  Any dtype.
 */
int sandy_hip_layout_transform(const SandyTensor* in, const SandyTensor* out, int32_t kind, void* stream,
                               char* err, size_t err_cap);

/* ---------------------------------------------------------------- MoE */

/* TopKKernelOp (replaces launch_cuda_topk, src/device/cuda/CudaTopKKernels.cu:
 * 616-646).  Order: value descending, index ascending on ties. */
int sandy_hip_topk(const SandyTensor* x, int64_t k, int64_t axis, const SandyTensor* values,
                   const SandyTensor* indices, void* stream, char* err, size_t err_cap);

/* MoeGatherKernelOp (replaces launch_cuda_moe_gather, src/device/cuda/
 * CudaGatherKernels.cu:389-649): stable permute, rows ordered expert, then
 * token, then slot (src/core/TensorCalc.cpp:1634-1660), computed on the
 * device with no host round trip. */
int sandy_hip_moe_gather(const SandyTensor* x, const SandyTensor* topk_ids,
                         const SandyTensor* topk_weights, int64_t num_experts, int64_t top_k,
                         const SandyTensor* packed_x, const SandyTensor* packed_weights,
                         const SandyTensor* token_ids, const SandyTensor* expert_offsets,
                         void* stream, char* err, size_t err_cap);

/* MoeMatMulKernelOp (replaces launch_cuda_moe_matmul, src/device/cuda/
 * CudaMatMulKernels.cu:294-616): grouped expert GEMM over expert_offsets, on
 * bf16 MFMA for bf16 operands. */
int sandy_hip_moe_matmul(const SandyTensor* x, const SandyTensor* expert_offsets,
                         const SandyTensor* weight, int32_t transpose_rhs, const SandyTensor* out,
                         void* stream, char* err, size_t err_cap);

/* MoeScatterSumKernelOp (replaces launch_cuda_moe_scatter_sum,
 * src/device/cuda/CudaMoeScatterSumKernels.cu:243-405): deterministic
 * per-token combine in packed-row order, no atomics. */
int sandy_hip_moe_scatter_sum(const SandyTensor* packed_out, const SandyTensor* packed_weights,
                              const SandyTensor* token_ids, const SandyTensor* out,
                              void* stream, char* err, size_t err_cap);

/* ---------------------------------------------------------------- dense matmul */

/* MatMulKernelOp (src/ir/KernelIR.h:447-471; replaces launch_cuda_matmul,
 * src/device/cuda/CudaMatMulKernels.cu:221-292, and its cuBLAS call at
 * 173-216).  lhs [.., M, K] (or [.., K, M] when transpose_lhs), rhs [.., K, N]
 * (or [.., N, K] when transpose_rhs), out [batch.., M, N]; batch dims
 * broadcast as in src/core/ShapeUtil.cpp:39-71 (1, equal, or a multiple:
 * grouped heads).  Same float dtype everywhere, contiguous views.  bf16 with
 * transpose_rhs runs on MFMA (fp32 accumulation); every other case keeps the
 * reference's per-output k order. */
int sandy_hip_matmul(const SandyTensor* lhs, const SandyTensor* rhs, int32_t transpose_lhs,
                     int32_t transpose_rhs, const SandyTensor* out, void* stream, char* err, size_t err_cap);

/* LinearKernelOp (src/ir/KernelIR.h:426-445; CPU semantics src/core/
 * TensorCalc.cpp:722-773 -- the reference's CUDA device rejects it,
 * src/device/cuda/CudaDevice.cpp:536-537): out[.., o] = bias[o] +
 * sum_i x[.., i] * weight[o, i]. */
/* Gated MLP input projection in one launch: out[.., m, i] = act(gate) * up
 * with gate = lhs . W[2i]^T and up = lhs . W[2i + 1]^T, each rounded to the
 * output dtype as sandy_hip_matmul stores it, then the SiLU (activation 1) or
 * GELU (2) scalar DAG of the element-wise group, fp32, rounded once.  rhs is
 * [2 ffn, k] with the gate and up rows interleaved; out is [.., m, ffn].
 * Bit-identical to sandy_hip_matmul (transpose_rhs) followed by
 * sandy_hip_elementwise.  bf16, k a multiple of 32, at most 64 rows (the
 * decode GEMM); otherwise SANDY_ERR_UNSUPPORTED.  Fuses the program's
 * gate/up __matmul pair and its __mul(__silu(gate), up) group
 * (src/models/tinyllama/common.sandy.go:3-5); the reference has no single
 * counterpart. */
int sandy_hip_matmul_glu(const SandyTensor* lhs, const SandyTensor* rhs, int32_t activation, const SandyTensor* out,
                         void* stream, char* err, size_t err_cap);

/*
 * Row statistics passed between the fused decode GEMMs below: sumsq points to
 * rows x parts float64 values, row-major, parts = ceil(cols / 16); value
 * [r, p] is the sum of the squares of row r's columns 16 p .. 16 p + 15 of
 * the matrix they describe (each square exact in float64, so their sum is the
 * RMSNorm's sum of squares, src/core/TensorCalc.cpp:1953-2000).
 */
typedef struct SandyRowStats {
    double* sumsq;
    int64_t rows;
    int64_t parts;
} SandyRowStats;

/* Decode projection with the residual add in its epilogue: out[m, n] =
 * bf16(residual[m, n] + bf16(sum_k lhs[m, k] * rhs[n, k])) -- bit-identical to
 * sandy_hip_matmul (transpose_rhs) followed by the residual add the program
 * writes next (__add(x, h), src/models/tinyllama/common.sandy.go:1-9) -- and,
 * when out_stats is given, out's row statistics for sandy_hip_matmul_rms.
 * bf16, lhs [m, k], rhs [n, k], k a multiple of 32, m <= 64; residual may be
 * out itself.  The reference runs the two ops separately; this fused form
 * has no single counterpart there. */
int sandy_hip_matmul_residual(const SandyTensor* lhs, const SandyTensor* rhs, const SandyTensor* residual,
                              const SandyTensor* out, const SandyRowStats* out_stats, void* stream, char* err,
                              size_t err_cap);

/* Decode projection of RMSNorm(lhs) * norm_weight: the normalised row is
 * formed in the GEMM's operand registers from lhs and its row statistics
 * (from sandy_hip_matmul_residual), with sandy_hip_norm's arithmetic (float64
 * sum of squares, float inverse 1 / sqrt(float(sum / k) + eps), y = x * inv *
 * w rounded once to bf16), so the result is bit-identical to sandy_hip_norm
 * followed by sandy_hip_matmul (activation 0) or sandy_hip_matmul_glu
 * (activation 1 / 2, rhs rows interleaved as there).  The reference's
 * __rms_norm + __matmul pair (src/models/tinyllama/common.sandy.go:1-9); no
 * single counterpart there. */
int sandy_hip_matmul_rms(const SandyTensor* lhs, const SandyRowStats* lhs_stats, const SandyTensor* norm_weight,
                         double eps, const SandyTensor* rhs, int32_t activation, const SandyTensor* out, void* stream,
                         char* err, size_t err_cap);
int sandy_hip_linear(const SandyTensor* x, const SandyTensor* weight, const SandyTensor* bias,
                     const SandyTensor* out, void* stream, char* err, size_t err_cap);

/*
 * Decode rows (1 to 4 of them) through the reference's fp32 chain
 *     out = [residual +] act(LinearKernelOp([NormKernelOp LayerNorm](x), weight, bias))
 * in one launch: the per-block op sequence of the GPT-2 program
 * (src/models/gpt2_small.sandy.go: ln_1 -> q/k/v, c_proj + residual,
 * ln_2 -> c_fc -> GELU, c_proj + residual; CPU arithmetic src/core/
 * TensorCalc.cpp layer_norm 2010-2077, linear 722-773, add 562-663, the GELU
 * of src/ir/BuiltinLowering.cpp:116-140).  x [..., k] f32 (rows = numel / k),
 * weight [n, k] f32, out [..., n]; ln_weight / ln_bias [k] (both or
 * neither: no LayerNorm), bias [n] or NULL, activation 0 (none) or 2
 * (GELU), residual like out or NULL.  The whole machine reads the weight in
 * one pass; the dot products sum in another order than the reference's k
 * loop (fp32 rounding, not bit for bit).  k a multiple of 4, rows * k <=
 * 16384; x and weight 16-byte aligned.
 */
int sandy_hip_decode_linear(const SandyTensor* x, const SandyTensor* ln_weight, const SandyTensor* ln_bias,
                            double eps, const SandyTensor* weight, const SandyTensor* bias, int32_t activation,
                            const SandyTensor* residual, const SandyTensor* out, void* stream, char* err,
                            size_t err_cap);

/* ---------------------------------------------------------------- safetensors weights
 *
 * EagerSafeTensorWeights (src/weight/SafeTensorWeights.h:29-48,
 * SafeTensorWeights.cpp:44-117): header parsing with the reference's dtype
 * table and error wording, tensors listed in name order (its descriptors()
 * order).  Instead of holding the file in host memory, the data section is
 * streamed through pinned staging buffers into one device arena in which
 * every tensor starts at a 256-byte-aligned arena_offset.  Host-only except
 * sandy_hip_safetensors_upload. */
typedef struct SandySafetensors SandySafetensors;

typedef struct SandySafetensorInfo {
    char name[256];
    int32_t dtype;                      /* SandyDType */
    int32_t rank;
    int64_t dims[SANDY_HIP_MAX_RANK];
    uint64_t file_offset;               /* within the data section */
    uint64_t nbytes;
    uint64_t arena_offset;              /* where sandy_hip_safetensors_upload puts it */
} SandySafetensorInfo;

int sandy_hip_safetensors_open(const char* path, SandySafetensors** out, char* err, size_t err_cap);
void sandy_hip_safetensors_close(SandySafetensors* st);
int64_t sandy_hip_safetensors_count(const SandySafetensors* st);
/* bytes of device memory the arena needs (sum of 256-aligned tensor sizes) */
uint64_t sandy_hip_safetensors_arena_bytes(const SandySafetensors* st);
int sandy_hip_safetensors_info(const SandySafetensors* st, int64_t index, SandySafetensorInfo* info, char* err,
                               size_t err_cap);
/* index of a tensor by name, -1 when absent (get_tensor returning null) */
int64_t sandy_hip_safetensors_find(const SandySafetensors* st, const char* name);
/* copies every tensor to arena + arena_offset (arena 256-byte aligned, at
 * least arena_bytes); returns when the copies are complete */
int sandy_hip_safetensors_upload(SandySafetensors* st, void* arena, uint64_t arena_bytes, void* stream, char* err,
                                 size_t err_cap);

/* ---------------------------------------------------------------- device runtime
 *
 * A HIP device object with the reference Device's responsibilities
 * (src/device/Device.h:27-66): buffers by id, paged tensor pools, stream and
 * graph capture.  A Device::run on top of it calls the kernel entry points
 * above with this object's stream and views.
 *
 * Paged pools keep their bookkeeping on the device: one pool allocation of
 * pages ([pages, prefix, page_size, inner], the reference's page layout), an
 * int32 block table [max_tensors, max_blocks] and int32 grow lengths
 * [max_tensors].  Appends are one kernel launch (the reference issues one
 * cudaMemcpyAsync per row, src/device/cuda/CudaPagedTensor.cpp:649-740), and
 * sandy_hip_device_paged_append_step reads positions on the device, so a whole
 * decode step (append + attention) can be captured in a HIP graph.
 */
typedef struct SandyHipDevice SandyHipDevice;

typedef struct SandyPagedPoolDesc {     /* DevicePagedPoolDesc, src/device/DeviceTypes.h:36-42 */
    int32_t dtype;
    int32_t rank;
    int64_t dims[SANDY_HIP_MAX_RANK];   /* template shape; dims[grow_dim] is ignored */
    int64_t grow_dim;
    int64_t page_size;                  /* power of two */
    int64_t initial_pages;
    int64_t max_pages;                  /* < 0: the pool grows on demand */
    int64_t max_tensors;                /* rows of the device block table */
    int64_t max_blocks;                 /* pages per tensor (block table columns) */
} SandyPagedPoolDesc;

typedef struct SandyPagedMeta {         /* DevicePagedTensorMeta, src/device/DeviceTypes.h:44-52 */
    uint32_t pool;
    int32_t dtype;
    int32_t rank;
    int32_t slot;                       /* row of the pool's block table */
    int64_t dims[SANDY_HIP_MAX_RANK];   /* logical shape (grow dim = grow_length) */
    int64_t grow_dim;
    int64_t page_size;
    int64_t grow_length;
    int64_t page_count;
    int64_t page_element_count;
} SandyPagedMeta;

/* Device lifetime.  The device owns one HIP stream (default priority). */
int sandy_hip_device_create(int32_t ordinal, SandyHipDevice** out, char* err, size_t err_cap);
void sandy_hip_device_destroy(SandyHipDevice* dev);
void* sandy_hip_device_stream(SandyHipDevice* dev);
int sandy_hip_device_synchronize(SandyHipDevice* dev, char* err, size_t err_cap);

/* Buffers (Device::alloc/dealloc/load/read).  load and read synchronise. */
int sandy_hip_device_alloc(SandyHipDevice* dev, uint64_t bytes, uint32_t* buffer, char* err, size_t err_cap);
int sandy_hip_device_dealloc(SandyHipDevice* dev, uint32_t buffer, char* err, size_t err_cap);
void* sandy_hip_device_buffer(SandyHipDevice* dev, uint32_t buffer);
int sandy_hip_device_load(SandyHipDevice* dev, const void* host, uint64_t bytes, uint32_t* buffer, char* err,
                          size_t err_cap);
int sandy_hip_device_read(SandyHipDevice* dev, uint32_t buffer, uint64_t offset, uint64_t bytes, void* host,
                          char* err, size_t err_cap);

/* Paged tensors (Device::createPagedPool .. destroyPagedPool). */
int sandy_hip_device_paged_pool_create(SandyHipDevice* dev, const SandyPagedPoolDesc* desc, uint32_t* pool,
                                       char* err, size_t err_cap);
int sandy_hip_device_paged_pool_destroy(SandyHipDevice* dev, uint32_t pool, char* err, size_t err_cap);
int sandy_hip_device_paged_alloc(SandyHipDevice* dev, uint32_t pool, uint32_t* tensor, char* err, size_t err_cap);
int sandy_hip_device_paged_dealloc(SandyHipDevice* dev, uint32_t tensor, char* err, size_t err_cap);
int sandy_hip_device_paged_reserve(SandyHipDevice* dev, uint32_t tensor, int64_t page_count, char* err,
                                   size_t err_cap);
/* Appends a dense chunk (logical shape with the grow dim = chunk length) in
 * one device copy; stream ordered, no host sync. */
int sandy_hip_device_paged_append(SandyHipDevice* dev, uint32_t tensor, const SandyTensor* chunk, char* err,
                                  size_t err_cap);
/* Appends one grow row to each of `count` tensors of one pool: rows is
 * [count, <template dims with the grow dim = 1>]; each tensor's position is
 * read from its device-side length, which the kernel advances.  Pages for the
 * new rows must already be reserved (sandy_hip_device_paged_reserve). */
int sandy_hip_device_paged_append_step(SandyHipDevice* dev, uint32_t pool, const uint32_t* tensors, int32_t count,
                                       const SandyTensor* rows, char* err, size_t err_cap);
/* The K and V step appends of one decode step in one launch: as two
 * sandy_hip_device_paged_append_step calls, (k_pool, k_tensors, k_rows) and
 * (v_pool, v_tensors, v_rows), for count <= 64 tensors each.  Every check runs
 * before any bookkeeping moves.  The two Engine::paged_append_op calls of a
 * decode step (src/engine/Engine.cpp:548-596, one per cache); the reference
 * has no single counterpart. */
int sandy_hip_device_paged_append_step_kv(SandyHipDevice* dev, uint32_t k_pool, const uint32_t* k_tensors,
                                          uint32_t v_pool, const uint32_t* v_tensors, int32_t count,
                                          const SandyTensor* k_rows, const SandyTensor* v_rows, char* err,
                                          size_t err_cap);
/* One decode step's q/k/v post-processing in one launch, for `count` <= 256
 * sequences: qkv is the [count, (q_heads + 2 kv_heads) head_dim] bf16 output
 * of the fused q/k/v projection.  q heads are rotated into q_out [count,
 * q_heads, 1, head_dim]; k heads are rotated and appended as the next row of
 * k_tensors[i] (pool k_pool), v heads appended to v_tensors[i] (v_pool), both
 * lengths advanced on the device.  RoPE as sandy_hip_rope with full rotary
 * (split_half or interleaved) and positions[i] for sequence i; appends as
 * sandy_hip_device_paged_append_step.  Fuses two RoPEKernelOps
 * (KernelIR.h:575-610) and two Engine::paged_append_op calls
 * (src/engine/Engine.cpp:548-596) of the TinyLlama eval_token program
 * (src/models/tinyllama/common.sandy.go:24-28); the
 * reference has no single counterpart. */
int sandy_hip_device_decode_qkv(SandyHipDevice* dev, uint32_t k_pool, const uint32_t* k_tensors, uint32_t v_pool,
                                const uint32_t* v_tensors, int32_t count, const SandyTensor* qkv, int32_t q_heads,
                                const SandyTensor* positions, double theta, int32_t split_half,
                                const SandyTensor* q_out, char* err, size_t err_cap);
/* The q/k/v projection of one decode step with sandy_hip_device_decode_qkv
 * in its epilogue: one launch for the GEMM, both RoPEs and both appends.
 * lhs [count, k] bf16 (count <= 64) is the block input; with lhs_stats and
 * norm_weight (both or neither) it is RMS-normalised first, as in
 * sandy_hip_matmul_rms.  rhs [(q_heads + 2 kv_heads) head_dim, k] is the
 * fused q/k/v weight; for split_half RoPE its q and k rows must be
 * pair-ordered within each head (row i of a head, then row i + head_dim / 2,
 * for i < head_dim / 2; v rows as they are).  Sequence i's row is appended at
 * row positions[i] of k_tensors[i] and v_tensors[i], whose device lengths must
 * equal positions[i] (as sandy_hip_device_paged_lengths returns them; a
 * mismatch sets SANDY_DEVERR_POSITION) and become positions[i] + 1.  Results
 * are bit-identical to sandy_hip_matmul_rms / sandy_hip_matmul into a qkv
 * buffer followed by sandy_hip_device_decode_qkv.  Fuses the q/k/v
 * MatMulKernelOp (src/ir/KernelIR.h), its two RoPEKernelOps (KernelIR.h:575-610)
 * and two Engine::paged_append_op calls (src/engine/Engine.cpp:548-596) of
 * the TinyLlama eval_token program (src/models/tinyllama/common.sandy.go:
 * 11-28); the reference has no single counterpart. */
int sandy_hip_device_matmul_qkv(SandyHipDevice* dev, const SandyTensor* lhs, const SandyRowStats* lhs_stats,
                                const SandyTensor* norm_weight, double eps, const SandyTensor* rhs, uint32_t k_pool,
                                const uint32_t* k_tensors, uint32_t v_pool, const uint32_t* v_tensors, int32_t count,
                                int32_t q_heads, const SandyTensor* positions, double theta, int32_t split_half,
                                const SandyTensor* q_out, char* err, size_t err_cap);
/* positions[i] = device length of tensors[i] - 1 (int32 or int64 output), for
 * the position_offsets of decode attention inside a captured step. */
int sandy_hip_device_paged_positions(SandyHipDevice* dev, uint32_t pool, const uint32_t* tensors, int32_t count,
                                     const SandyTensor* positions, char* err, size_t err_cap);
/* lengths[i] = device length of tensors[i]: the position the next appended
 * row takes (the position_id of a decode step, computed inside the step). */
int sandy_hip_device_paged_lengths(SandyHipDevice* dev, uint32_t pool, const uint32_t* tensors, int32_t count,
                                   const SandyTensor* lengths, char* err, size_t err_cap);
int sandy_hip_device_paged_meta(SandyHipDevice* dev, uint32_t tensor, SandyPagedMeta* meta, char* err,
                                size_t err_cap);
/* Reads the dense logical tensor (Device::read(DevicePagedTensorView)); synchronises. */
int sandy_hip_device_paged_read(SandyHipDevice* dev, uint32_t tensor, void* host, uint64_t bytes, char* err,
                                size_t err_cap);
/* The pool as a SandyPagedCache, its block table [max_tensors, max_blocks]
 * int32 and grow lengths [max_tensors] int32 (device-resident views). */
int sandy_hip_device_paged_views(SandyHipDevice* dev, uint32_t pool, SandyPagedCache* cache,
                                 SandyTensor* block_table, SandyTensor* lengths, char* err, size_t err_cap);
/* Re-reads the device lengths into the host bookkeeping (after graph replays). */
int sandy_hip_device_paged_sync(SandyHipDevice* dev, uint32_t pool, char* err, size_t err_cap);

/* HIP graph capture of work on the device stream. */
int sandy_hip_device_graph_begin(SandyHipDevice* dev, char* err, size_t err_cap);
int sandy_hip_device_graph_end(SandyHipDevice* dev, uint32_t* graph, char* err, size_t err_cap);
int sandy_hip_device_graph_launch(SandyHipDevice* dev, uint32_t graph, char* err, size_t err_cap);
int sandy_hip_device_graph_destroy(SandyHipDevice* dev, uint32_t graph, char* err, size_t err_cap);

#ifdef __cplusplus
}
#endif

#endif
