/*
 * sandy_oracle.h -- CPU restatement of SandyRT's reference CPU math for the
 * hot path (fused element-wise groups, norms, RoPE, softmax, decode attention,
 * top-k and the MoE dispatch/combine chain).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * backend; it is linked by tests/, by __graft_entry__.smoke() and by the
 * cpu_baseline leg of bench.py, and by nothing on the product path.
 *
 * Every function follows one reference function and cites it (file:line under
 * the reference tree).  All tensors are dense row-major; float tensors are
 * F32 or BF16 (bf16 stored as uint16 bit patterns, converted with
 * round-to-nearest-even exactly as src/core/Tensor.h:43-49), index tensors are
 * I32 or I64.  Arithmetic order and accumulation types (float vs double) are
 * kept identical to the reference so that results agree bit-for-bit with the
 * reference build when both use the same libm.
 *
 * Every function returns 0 on success or -1 on error; the message (worded
 * like the reference's) is available from oracle_last_error().
 */
#ifndef SANDY_ORACLE_H
#define SANDY_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes follow the order of sandy::core::DType (src/core/Tensor.h:13) */
enum { OR_F32 = 0, OR_F16 = 1, OR_BF16 = 2, OR_I32 = 3, OR_I64 = 4, OR_U8 = 5 };

/* scalar op codes follow sandy::ir::kernel_ir::ScalarOp (src/ir/KernelIR.h:317-337) */
enum {
    OR_SC_LOAD = 0, OR_SC_CONST, OR_SC_ADD, OR_SC_SUB, OR_SC_MUL, OR_SC_DIV,
    OR_SC_MAX, OR_SC_MIN, OR_SC_NEG, OR_SC_SQRT, OR_SC_RSQRT, OR_SC_EXP,
    OR_SC_LOG, OR_SC_TANH, OR_SC_RELU, OR_SC_CAST
};

typedef struct OracleScalarNode {
    uint32_t id;
    int32_t op;
    int32_t dtype;
    uint32_t input_index;
    double constant;
    int32_t operand_count;
    uint32_t operands[2];
} OracleScalarNode;

const char* oracle_last_error(void);

uint16_t oracle_bf16_from_float(float v);
float oracle_bf16_to_float(uint16_t bits);
void oracle_f32_to_bf16(const float* src, uint16_t* dst, int64_t n);
void oracle_bf16_to_f32(const uint16_t* src, float* dst, int64_t n);

int oracle_rms_norm(const void* x, const void* weight, void* out, int dtype,
                    int64_t rows, int64_t cols, float eps);
int oracle_layer_norm(const void* x, const void* weight, const void* bias, void* out,
                      int dtype, int64_t rows, int64_t cols, float eps);
int oracle_softmax(const void* x, void* out, int dtype,
                   int64_t outer, int64_t axis, int64_t inner);
int oracle_sum(const void* x, void* out, int dtype,
               int64_t outer, int64_t axis, int64_t inner);
int oracle_rope(const void* x, const void* position_ids, int pos_dtype, int64_t pos_count,
                void* out, int dtype, int64_t vectors, int64_t seq, int64_t dim,
                float theta, int64_t rotary_dim, int split_half);
int oracle_attention(const void* q, const void* k, const void* v,
                     const void* position_offsets, int pos_dtype, void* out, int dtype,
                     int64_t batch, int64_t heads, int64_t kv_heads, int64_t tq, int64_t tk,
                     int64_t head_dim, int64_t window, float scale);
int oracle_topk(const void* x, void* values, void* indices, int idx_dtype, int dtype,
                int64_t outer, int64_t axis, int64_t inner, int64_t k);
int oracle_embedding(const void* ids, int ids_dtype, int64_t n_ids, const void* weight,
                     int dtype, int64_t vocab, int64_t hidden, void* out);
int oracle_moe_gather(const void* x, int dtype, const void* topk_ids, int ids_dtype,
                      const void* topk_weights, int w_dtype,
                      int64_t batch, int64_t seq, int64_t hidden,
                      int64_t num_experts, int64_t top_k,
                      void* packed_x, void* packed_weights,
                      void* token_ids, int tok_dtype, void* expert_offsets, int off_dtype);
int oracle_moe_matmul(const void* x, const void* expert_offsets, int off_dtype,
                      const void* weight, int dtype, int64_t batch, int64_t rows,
                      int64_t in_features, int64_t experts, int64_t out_features,
                      int transpose_rhs, void* out);
int oracle_moe_scatter_sum(const void* packed_out, const void* packed_weights,
                           const void* token_ids, int tok_dtype, int dtype,
                           int64_t batch, int64_t rows, int64_t hidden, int64_t seq,
                           void* out);
int oracle_matmul(const void* lhs, const int64_t* ldims, int lrank, const void* rhs, const int64_t* rdims,
                  int rrank, int transpose_lhs, int transpose_rhs, void* out, int dtype);
int oracle_linear(const void* x, const void* weight, const void* bias, void* out, int dtype,
                  int64_t rows, int64_t in_features, int64_t out_features);

/* unfused single element-wise ops: 0 add, 1 mul, 2 div (binary, right-aligned
 * broadcast of shapes); 10 relu, 11 sqrt, 12 tanh (unary) */
int oracle_binary(int op, const void* lhs, const int64_t* lshape, int lrank,
                  const void* rhs, const int64_t* rshape, int rrank,
                  void* out, const int64_t* oshape, int orank, int dtype);
int oracle_unary(int op, const void* x, void* out, int dtype, int64_t n);

/* one fused element-wise group: the scalar DAG evaluated per element in fp32
 * registers (inputs[i] has input_numels[i] elements; broadcast[i] = 1 means
 * right-aligned broadcast, index = linear % numel) */
int oracle_elementwise_dag(const OracleScalarNode* nodes, int32_t node_count, uint32_t result,
                           const void* const* inputs, const int32_t* input_dtypes,
                           const int64_t* input_numels, const int32_t* broadcast,
                           int32_t input_count, void* out, int out_dtype, int64_t numel);

/* paged storage -> dense logical tensor (page = [prefix, page_size, inner]) */
int oracle_paged_to_dense(const void* pool, int64_t page_elements, const int32_t* page_ids,
                          int64_t page_count, int64_t prefix, int64_t grow_length,
                          int64_t page_size, int64_t inner, int64_t elem_size, void* out);

#ifdef __cplusplus
}
#endif

#endif
