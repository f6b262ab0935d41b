/*
 * sandy_oracle.c -- CPU restatement of the reference CPU math (TEST
 * INFRASTRUCTURE ONLY; see sandy_oracle.h).
 *
 * Reference: src/core/TensorCalc.cpp (TensorCalc), src/core/Tensor.h (bf16),
 * src/device/cpu/CpuDevice.cpp (paged read), src/device/cuda/
 * CudaElementwiseKernels.cu (fused scalar-DAG semantics).  Each function names
 * the lines it follows.  Loops, accumulation types and the order of float
 * operations are the reference's, so that a build against the same libm gives
 * bit-identical results.  Compile without -ffast-math and without FMA
 * contraction (-ffp-contract=off) so the float expression order is kept.
 */
#include "sandy_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_err[256];

static int fail(const char* msg) {
    snprintf(g_err, sizeof(g_err), "%s", msg);
    return -1;
}

const char* oracle_last_error(void) { return g_err; }

/* src/core/Tensor.h:36-49 -- bf16 <-> f32, RNE with (bits + 0x7fff + lsb) >> 16 */
uint16_t oracle_bf16_from_float(float v) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    uint32_t lsb = (bits >> 16) & 1u;
    return (uint16_t)((bits + 0x7fffu + lsb) >> 16);
}

float oracle_bf16_to_float(uint16_t b) {
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void oracle_f32_to_bf16(const float* src, uint16_t* dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = oracle_bf16_from_float(src[i]);
}

void oracle_bf16_to_f32(const uint16_t* src, float* dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = oracle_bf16_to_float(src[i]);
}

/* TensorCalc.cpp:29-47 load_f32/store_f32/load_bf16/store_bf16 */
static inline float ld(const void* p, int dtype, int64_t i) {
    if (dtype == OR_BF16) return oracle_bf16_to_float(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

static inline void st(void* p, int dtype, int64_t i, float v) {
    if (dtype == OR_BF16)
        ((uint16_t*)p)[i] = oracle_bf16_from_float(v);
    else
        ((float*)p)[i] = v;
}

static int is_float(int dtype) { return dtype == OR_F32 || dtype == OR_BF16; }
static int is_index(int dtype) { return dtype == OR_I32 || dtype == OR_I64; }

/* TensorCalc.cpp:159-170 read_index / 172-182 store_index (i32 narrows) */
static inline int64_t ld_idx(const void* p, int dtype, int64_t i) {
    if (dtype == OR_I32) return ((const int32_t*)p)[i];
    return ((const int64_t*)p)[i];
}

static inline void st_idx(void* p, int dtype, int64_t i, int64_t v) {
    if (dtype == OR_I32)
        ((int32_t*)p)[i] = (int32_t)v;
    else
        ((int64_t*)p)[i] = v;
}

/* TensorCalc.cpp:1953-2000 rms_norm_impl: double sum of squares, float invRms,
 * out = x * invRms * w evaluated left to right in float */
int oracle_rms_norm(const void* x, const void* weight, void* out, int dtype,
                    int64_t rows, int64_t cols, float eps) {
    if (!is_float(dtype)) return fail("rms_norm input unsupported dtype");
    if (cols < 0) return fail("rms_norm hidden dimension must be static");
    for (int64_t r = 0; r < rows; r++) {
        double square_sum = 0.0;
        int64_t base = r * cols;
        for (int64_t c = 0; c < cols; c++) {
            float xv = ld(x, dtype, base + c);
            square_sum += (double)xv * (double)xv;
        }
        float inv_rms = 1.0f / sqrtf((float)(square_sum / (double)cols) + eps);
        for (int64_t c = 0; c < cols; c++) {
            float xv = ld(x, dtype, base + c);
            float wv = weight ? ld(weight, dtype, c) : 1.0f;
            float y = xv * inv_rms;
            y = y * wv;
            st(out, dtype, base + c, y);
        }
    }
    return 0;
}

/* TensorCalc.cpp:2010-2077 layer_norm: double mean, double variance of
 * (double)x - mean, float invStd, out = (x - (float)mean) * invStd * w + b */
int oracle_layer_norm(const void* x, const void* weight, const void* bias, void* out,
                      int dtype, int64_t rows, int64_t cols, float eps) {
    if (!is_float(dtype)) return fail("layer_norm input unsupported dtype");
    for (int64_t r = 0; r < rows; r++) {
        int64_t base = r * cols;
        double mean = 0.0;
        for (int64_t i = 0; i < cols; i++) mean += (double)ld(x, dtype, base + i);
        mean /= (double)cols;
        double variance = 0.0;
        for (int64_t i = 0; i < cols; i++) {
            double centered = (double)ld(x, dtype, base + i) - mean;
            variance += centered * centered;
        }
        variance /= (double)cols;
        float inv_std = 1.0f / sqrtf((float)variance + eps);
        for (int64_t i = 0; i < cols; i++) {
            float centered = ld(x, dtype, base + i) - (float)mean;
            float v = centered * inv_std;
            v = v * ld(weight, dtype, i);
            v = v + ld(bias, dtype, i);
            st(out, dtype, base + i, v);
        }
    }
    return 0;
}

/* TensorCalc.cpp:1337-1399 softmax over one axis: float max, all -inf -> 0,
 * double sum of float exp(x - max), float invSum = 1 / (float)sum */
int oracle_softmax(const void* x, void* out, int dtype,
                   int64_t outer, int64_t axis, int64_t inner) {
    if (!is_float(dtype)) return fail("softmax input unsupported dtype");
    for (int64_t o = 0; o < outer; o++) {
        for (int64_t i = 0; i < inner; i++) {
            int64_t base = o * axis * inner + i;
            float max_value = -INFINITY;
            for (int64_t a = 0; a < axis; a++) {
                float v = ld(x, dtype, base + a * inner);
                if (max_value < v) max_value = v; /* std::max(max, v) */
            }
            if (isinf(max_value) && max_value < 0.0f) {
                for (int64_t a = 0; a < axis; a++) st(out, dtype, base + a * inner, 0.0f);
                continue;
            }
            double sum = 0.0;
            for (int64_t a = 0; a < axis; a++)
                sum += (double)expf(ld(x, dtype, base + a * inner) - max_value);
            float inv_sum = 1.0f / (float)sum;
            for (int64_t a = 0; a < axis; a++) {
                float v = expf(ld(x, dtype, base + a * inner) - max_value) * inv_sum;
                st(out, dtype, base + a * inner, v);
            }
        }
    }
    return 0;
}

/* TensorCalc.cpp:1401-1445 sum over one axis, float accumulation in axis order */
int oracle_sum(const void* x, void* out, int dtype, int64_t outer, int64_t axis, int64_t inner) {
    if (!is_float(dtype)) return fail("sum input unsupported dtype");
    if (axis <= 0) return fail("sum axis dimension must be static and positive");
    for (int64_t o = 0; o < outer; o++) {
        for (int64_t i = 0; i < inner; i++) {
            float acc = 0.0f;
            int64_t base = o * axis * inner + i;
            for (int64_t a = 0; a < axis; a++) acc += ld(x, dtype, base + a * inner);
            st(out, dtype, o * inner + i, acc);
        }
    }
    return 0;
}

/* TensorCalc.cpp:1823-1937 rope_impl.  Position of vector v is v % seq, or
 * read from position_ids (numel 1: id[0] + v % seq; numel == vectors: id[v];
 * numel == seq: id[v % seq]).  Split-half pairs (i, half + i) with angle
 * pos / powf(theta, 2i / dim); interleaved pairs (2i, 2i+1) with angle
 * pos / powf(theta, 2i / rotary_dim).  Un-rotated tail copied. */
int oracle_rope(const void* x, const void* position_ids, int pos_dtype, int64_t pos_count,
                void* out, int dtype, int64_t vectors, int64_t seq, int64_t dim,
                float theta, int64_t rotary_dim, int split_half) {
    if (!is_float(dtype)) return fail("rope input unsupported dtype");
    if (position_ids && !is_index(pos_dtype)) return fail("rope position_ids must be i32 or i64");
    if (theta <= 0.0f) return fail("rope theta must be > 0");
    if (dim <= 0 || dim % 2 != 0) return fail("rope last dimension must be positive and even");
    if (rotary_dim < 0) rotary_dim = dim;
    if (rotary_dim <= 0 || rotary_dim % 2 != 0) return fail("rope rotary_dim must be positive and even");
    if (rotary_dim > dim) return fail("rope rotary_dim must be <= last dimension");
    if (position_ids && pos_count != 1 && pos_count != seq && pos_count != vectors)
        return fail("rope position_ids numel must be 1, sequence length, or vector count");
    for (int64_t vec = 0; vec < vectors; vec++) {
        int64_t seq_pos = vec % seq;
        int64_t position = seq_pos;
        if (position_ids) {
            if (pos_count == 1)
                position = ld_idx(position_ids, pos_dtype, 0) + seq_pos;
            else if (pos_count == vectors)
                position = ld_idx(position_ids, pos_dtype, vec);
            else
                position = ld_idx(position_ids, pos_dtype, seq_pos);
            if (position < 0) return fail("rope position_ids must be non-negative");
        }
        int64_t base = vec * dim;
        if (split_half) {
            int64_t half = dim / 2;
            int64_t pairs = rotary_dim / 2;
            for (int64_t p = 0; p < pairs; p++) {
                float angle = (float)position / powf(theta, (float)(2 * p) / (float)dim);
                float c = cosf(angle);
                float s = sinf(angle);
                float first = ld(x, dtype, base + p);
                float second = ld(x, dtype, base + half + p);
                float a = first * c;
                float b = second * s;
                st(out, dtype, base + p, a - b);
                a = first * s;
                b = second * c;
                st(out, dtype, base + half + p, a + b);
            }
            for (int64_t i = pairs; i < half; i++) {
                st(out, dtype, base + i, ld(x, dtype, base + i));
                st(out, dtype, base + half + i, ld(x, dtype, base + half + i));
            }
        } else {
            for (int64_t p = 0; p < rotary_dim / 2; p++) {
                float angle = (float)position / powf(theta, (float)(2 * p) / (float)rotary_dim);
                float c = cosf(angle);
                float s = sinf(angle);
                float even = ld(x, dtype, base + 2 * p);
                float odd = ld(x, dtype, base + 2 * p + 1);
                float a = even * c;
                float b = odd * s;
                st(out, dtype, base + 2 * p, a - b);
                a = even * s;
                b = odd * c;
                st(out, dtype, base + 2 * p + 1, a + b);
            }
            for (int64_t i = rotary_dim; i < dim; i++) st(out, dtype, base + i, ld(x, dtype, base + i));
        }
    }
    return 0;
}

/* TensorCalc.cpp:1167-1314 attention_impl (rank-4 layout [B, H, T, D]; rank 3
 * is batch 1).  Query qi of batch b sits at position offsets[b] + qi; keys
 * ki > position or ki < position + 1 - window (window > 0) are masked.  Float
 * scores = (sum_d q*k) * scale, float max, double sum of exp((double)(s - max)),
 * float invSum, out[d] = sum_k (expf(s - max) * invSum) * v in key order. */
int oracle_attention(const void* q, const void* k, const void* v,
                     const void* position_offsets, int pos_dtype, void* out, int dtype,
                     int64_t batch, int64_t heads, int64_t kv_heads, int64_t tq, int64_t tk,
                     int64_t head_dim, int64_t window, float scale) {
    if (!is_float(dtype)) return fail("attention q unsupported dtype");
    if (window < 0) return fail("attention window must be >= 0");
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0)
        return fail("attention heads must be divisible by kv_heads");
    if (position_offsets && !is_index(pos_dtype))
        return fail("attention position_offsets must be i32 or i64");
    int64_t per_kv = heads / kv_heads;
    if (scale <= 0.0f) scale = 1.0f / sqrtf((float)head_dim);
    float* scores = (float*)malloc(sizeof(float) * (size_t)(tk > 0 ? tk : 1));
    for (int64_t b = 0; b < batch; b++) {
        int64_t base_pos = 0;
        if (position_offsets) {
            base_pos = ld_idx(position_offsets, pos_dtype, b);
            if (base_pos < 0) {
                free(scores);
                return fail("attention position_offsets must be non-negative");
            }
        }
        for (int64_t h = 0; h < heads; h++) {
            int64_t kh = h / per_kv;
            for (int64_t qi = 0; qi < tq; qi++) {
                int64_t qpos = base_pos + qi;
                int64_t min_key = 0;
                if (window > 0) {
                    min_key = qpos + 1 - window;
                    if (min_key < 0) min_key = 0;
                }
                float max_score = -INFINITY;
                for (int64_t ki = 0; ki < tk; ki++) {
                    float score = -INFINITY;
                    if (ki <= qpos && ki >= min_key) {
                        float acc = 0.0f;
                        for (int64_t d = 0; d < head_dim; d++) {
                            int64_t qidx = ((b * heads + h) * tq + qi) * head_dim + d;
                            int64_t kidx = ((b * kv_heads + kh) * tk + ki) * head_dim + d;
                            float prod = ld(q, dtype, qidx) * ld(k, dtype, kidx);
                            acc += prod;
                        }
                        score = acc * scale;
                    }
                    scores[ki] = score;
                    if (score > max_score) max_score = score;
                }
                double sum = 0.0;
                if (!(isinf(max_score) && max_score < 0.0f)) {
                    for (int64_t ki = 0; ki < tk; ki++)
                        sum += exp((double)(scores[ki] - max_score));
                }
                for (int64_t d = 0; d < head_dim; d++) {
                    float acc = 0.0f;
                    if (sum != 0.0) {
                        float inv_sum = 1.0f / (float)sum;
                        for (int64_t ki = 0; ki < tk; ki++) {
                            float s = scores[ki];
                            if (isinf(s) && s < 0.0f) continue;
                            float prob = expf(s - max_score) * inv_sum;
                            int64_t vidx = ((b * kv_heads + kh) * tk + ki) * head_dim + d;
                            float prod = prob * ld(v, dtype, vidx);
                            acc += prod;
                        }
                    }
                    st(out, dtype, ((b * heads + h) * tq + qi) * head_dim + d, acc);
                }
            }
        }
    }
    free(scores);
    return 0;
}

/* TensorCalc.cpp:1447-1518 topk: partial sort by (value desc, index asc); a
 * selection sort over the first k positions gives the same first k items. */
int oracle_topk(const void* x, void* values, void* indices, int idx_dtype, int dtype,
                int64_t outer, int64_t axis, int64_t inner, int64_t k) {
    if (!is_float(dtype)) return fail("topk input unsupported dtype");
    if (k <= 0) return fail("topk k must be > 0");
    if (axis <= 0 || k > axis) return fail("topk invalid k or axis dimension");
    if (!is_index(idx_dtype)) return fail("topk indices output shape or dtype mismatch");
    float* vals = (float*)malloc(sizeof(float) * (size_t)axis);
    int64_t* ids = (int64_t*)malloc(sizeof(int64_t) * (size_t)axis);
    for (int64_t o = 0; o < outer; o++) {
        for (int64_t i = 0; i < inner; i++) {
            int64_t base = o * axis * inner + i;
            for (int64_t a = 0; a < axis; a++) {
                vals[a] = ld(x, dtype, base + a * inner);
                ids[a] = a;
            }
            for (int64_t r = 0; r < k; r++) {
                int64_t best = r;
                for (int64_t a = r + 1; a < axis; a++) {
                    int better = vals[a] != vals[best] ? vals[a] > vals[best] : ids[a] < ids[best];
                    if (better) best = a;
                }
                float tv = vals[r]; vals[r] = vals[best]; vals[best] = tv;
                int64_t ti = ids[r]; ids[r] = ids[best]; ids[best] = ti;
                int64_t oi = o * k * inner + r * inner + i;
                st(values, dtype, oi, vals[r]);
                st_idx(indices, idx_dtype, oi, ids[r]);
            }
        }
    }
    free(vals);
    free(ids);
    return 0;
}

/* TensorCalc.cpp:1520-1563 embedding: out[i, :] = weight[ids[i], :] */
int oracle_embedding(const void* ids, int ids_dtype, int64_t n_ids, const void* weight,
                     int dtype, int64_t vocab, int64_t hidden, void* out) {
    if (!is_index(ids_dtype)) return fail("embedding ids must be i32 or i64");
    if (!is_float(dtype)) return fail("embedding weight unsupported dtype");
    for (int64_t i = 0; i < n_ids; i++) {
        int64_t t = ld_idx(ids, ids_dtype, i);
        if (t < 0 || t >= vocab) return fail("embedding id out of range");
        for (int64_t h = 0; h < hidden; h++) st(out, dtype, i * hidden + h, ld(weight, dtype, t * hidden + h));
    }
    return 0;
}

/* TensorCalc.cpp:1565-1667 moe_gather: rows ordered expert-major, then token,
 * then slot; expert_offsets[e] = first row of expert e, [E] = seq * top_k. */
int oracle_moe_gather(const void* x, int dtype, const void* topk_ids, int ids_dtype,
                      const void* topk_weights, int w_dtype,
                      int64_t batch, int64_t seq, int64_t hidden,
                      int64_t num_experts, int64_t top_k,
                      void* packed_x, void* packed_weights,
                      void* token_ids, int tok_dtype, void* expert_offsets, int off_dtype) {
    if (!is_float(dtype)) return fail("moe_gather x unsupported dtype");
    if (!is_float(w_dtype)) return fail("moe_gather topk_weights unsupported dtype");
    if (!is_index(ids_dtype)) return fail("moe_gather topk_ids must be i32 or i64");
    if (!is_index(tok_dtype)) return fail("moe_gather token_ids must be i32 or i64");
    if (!is_index(off_dtype)) return fail("moe_gather expert_offsets must be i32 or i64");
    if (num_experts <= 0 || top_k <= 0) return fail("moe_gather num_experts and top_k must be positive");
    int64_t rows = seq * top_k;
    for (int64_t b = 0; b < batch; b++) {
        int64_t row = 0;
        int64_t xb = b * seq * hidden, rb = b * seq * top_k, pb = b * rows * hidden;
        int64_t mb = b * rows, ob = b * (num_experts + 1);
        for (int64_t e = 0; e < num_experts; e++) {
            st_idx(expert_offsets, off_dtype, ob + e, row);
            for (int64_t t = 0; t < seq; t++) {
                for (int64_t s = 0; s < top_k; s++) {
                    int64_t ri = rb + t * top_k + s;
                    int64_t re = ld_idx(topk_ids, ids_dtype, ri);
                    if (re < 0 || re >= num_experts) return fail("moe_gather topk expert id out of range");
                    if (re != e) continue;
                    for (int64_t h = 0; h < hidden; h++)
                        st(packed_x, dtype, pb + row * hidden + h, ld(x, dtype, xb + t * hidden + h));
                    st(packed_weights, w_dtype, mb + row, ld(topk_weights, w_dtype, ri));
                    st_idx(token_ids, tok_dtype, mb + row, t);
                    row++;
                }
            }
        }
        st_idx(expert_offsets, off_dtype, ob + num_experts, row);
        if (row != rows) return fail("moe_gather routed row count mismatch");
    }
    return 0;
}

/* TensorCalc.cpp:1669-1743 moe_matmul: for rows [off[e], off[e+1]) of expert
 * e, out[row, o] = sum_i x[row, i] * W[e] (W[e] is [M, K] when transpose_rhs,
 * else [K, M]); float accumulation in i order. */
int oracle_moe_matmul(const void* x, const void* expert_offsets, int off_dtype,
                      const void* weight, int dtype, int64_t batch, int64_t rows,
                      int64_t in_features, int64_t experts, int64_t out_features,
                      int transpose_rhs, void* out) {
    if (!is_float(dtype)) return fail("moe_matmul x unsupported dtype");
    if (!is_index(off_dtype)) return fail("moe_matmul expert_offsets must be i32 or i64");
    for (int64_t b = 0; b < batch; b++) {
        int64_t ob = b * (experts + 1), xb = b * rows * in_features, yb = b * rows * out_features;
        for (int64_t e = 0; e < experts; e++) {
            int64_t begin = ld_idx(expert_offsets, off_dtype, ob + e);
            int64_t end = ld_idx(expert_offsets, off_dtype, ob + e + 1);
            if (begin < 0 || end < begin || end > rows) return fail("moe_matmul invalid expert offsets");
            for (int64_t r = begin; r < end; r++) {
                for (int64_t o = 0; o < out_features; o++) {
                    float acc = 0.0f;
                    for (int64_t i = 0; i < in_features; i++) {
                        float xv = ld(x, dtype, xb + r * in_features + i);
                        int64_t wi = transpose_rhs ? (e * out_features + o) * in_features + i
                                                   : (e * in_features + i) * out_features + o;
                        float prod = xv * ld(weight, dtype, wi);
                        acc += prod;
                    }
                    st(out, dtype, yb + r * out_features + o, acc);
                }
            }
        }
    }
    return 0;
}

/* TensorCalc.cpp:1745-1811 moe_scatter_sum: out zeroed, then for each packed
 * row in order: out[token] = store(load(out[token]) + w * packed[row]) -- the
 * accumulator is re-rounded to the output dtype after every add. */
int oracle_moe_scatter_sum(const void* packed_out, const void* packed_weights,
                           const void* token_ids, int tok_dtype, int dtype,
                           int64_t batch, int64_t rows, int64_t hidden, int64_t seq,
                           void* out) {
    if (!is_float(dtype)) return fail("moe_scatter_sum packed_out unsupported dtype");
    if (!is_index(tok_dtype)) return fail("moe_scatter_sum token_ids must be i32 or i64");
    for (int64_t i = 0; i < batch * seq * hidden; i++) st(out, dtype, i, 0.0f);
    for (int64_t b = 0; b < batch; b++) {
        int64_t pb = b * rows * hidden, mb = b * rows, ob = b * seq * hidden;
        for (int64_t r = 0; r < rows; r++) {
            int64_t t = ld_idx(token_ids, tok_dtype, mb + r);
            if (t < 0 || t >= seq) return fail("moe_scatter_sum token id out of range");
            float w = ld(packed_weights, dtype, mb + r);
            for (int64_t h = 0; h < hidden; h++) {
                int64_t dst = ob + t * hidden + h;
                float acc = ld(out, dtype, dst);
                float prod = w * ld(packed_out, dtype, pb + r * hidden + h);
                acc += prod;
                st(out, dtype, dst, acc);
            }
        }
    }
    return 0;
}

/* ShapeUtil.cpp:39-71 matmul_batch_shape: right-aligned; equal dims, a 1, or
 * one dim a multiple of the other (grouped heads) */
static int batch_shape(const int64_t* l, int lr, const int64_t* r, int rr, int64_t* out) {
    int orank = lr > rr ? lr : rr;
    for (int i = 0; i < orank; i++) {
        int li = lr - 1 - i, ri = rr - 1 - i;
        int64_t a = li >= 0 ? l[li] : 1, b = ri >= 0 ? r[ri] : 1, o;
        if (a == b) o = a;
        else if (a == 1) o = b;
        else if (b == 1) o = a;
        else if (a > b && a % b == 0) o = a;
        else if (b > a && b % a == 0) o = b;
        else return -1;
        out[orank - 1 - i] = o;
    }
    return orank;
}

/* TensorCalc.cpp:213-240 matmul_batch_offset: a source dim of 1 broadcasts; a
 * smaller source dim d serves batch/d consecutive output coordinates */
static int64_t batch_offset(int64_t index, const int64_t* bshape, int brank, const int64_t* sdims, int srank) {
    int sb = srank - 2;
    if (sb <= 0) return 0;
    int64_t strides[16], s = 1;
    for (int d = srank - 1; d >= 0; d--) {
        strides[d] = s;
        s *= sdims[d];
    }
    int64_t off = 0, rem = index;
    int shift = brank - sb;
    for (int bd = brank - 1; bd >= 0; bd--) {
        int64_t dim = bshape[bd], coord = rem % dim;
        rem /= dim;
        int sd = bd - shift;
        if (sd < 0 || sdims[sd] == 1) continue;
        if (sdims[sd] != dim) coord /= dim / sdims[sd];
        off += coord * strides[sd];
    }
    return off;
}

/* TensorCalc.cpp:804-919 matmul (plain loop path): for every output batch,
 * out[m, n] = sum over k in order of lhs[m, k] * rhs[k, n] (operands read
 * transposed when asked), float accumulation, row-major contiguous operands
 * of rank >= 2 */
int oracle_matmul(const void* lhs, const int64_t* ldims, int lrank, const void* rhs, const int64_t* rdims,
                  int rrank, int transpose_lhs, int transpose_rhs, void* out, int dtype) {
    if (!is_float(dtype)) return fail("matmul lhs unsupported dtype");
    if (lrank < 2) return fail("matmul lhs must have rank >= 2");
    if (rrank < 2) return fail("matmul rhs must have rank >= 2");
    if (lrank > 14 || rrank > 14) return fail("matmul rank too large");
    int64_t m = ldims[lrank - (transpose_lhs ? 1 : 2)], lk = ldims[lrank - (transpose_lhs ? 2 : 1)];
    int64_t rk = rdims[rrank - (transpose_rhs ? 1 : 2)], n = rdims[rrank - (transpose_rhs ? 2 : 1)];
    if (lk != rk) return fail("matmul contracting dimension mismatch");
    int64_t bshape[16];
    int brank = batch_shape(ldims, lrank - 2, rdims, rrank - 2, bshape);
    if (brank < 0) return fail("cannot broadcast matmul batch shapes");
    int64_t batches = 1;
    for (int i = 0; i < brank; i++) batches *= bshape[i];
    int64_t lrs = ldims[lrank - 1], rrs = rdims[rrank - 1];  /* row strides */
    for (int64_t b = 0; b < batches; b++) {
        int64_t lb = batch_offset(b, bshape, brank, ldims, lrank);
        int64_t rb = batch_offset(b, bshape, brank, rdims, rrank);
        int64_t ob = b * m * n;
        for (int64_t r = 0; r < m; r++) {
            for (int64_t c = 0; c < n; c++) {
                float acc = 0.0f;
                for (int64_t i = 0; i < lk; i++) {
                    int64_t li = transpose_lhs ? i * lrs + r : r * lrs + i;
                    int64_t ri = transpose_rhs ? c * rrs + i : i * rrs + c;
                    float prod = ld(lhs, dtype, lb + li) * ld(rhs, dtype, rb + ri);
                    acc += prod;
                }
                st(out, dtype, ob + r * n + c, acc);
            }
        }
    }
    return 0;
}

/* TensorCalc.cpp:722-773 linear: acc starts at bias[o], += x * w in i order */
int oracle_linear(const void* x, const void* weight, const void* bias, void* out, int dtype,
                  int64_t rows, int64_t in_features, int64_t out_features) {
    if (!is_float(dtype)) return fail("linear input unsupported dtype");
    for (int64_t b = 0; b < rows; b++) {
        for (int64_t o = 0; o < out_features; o++) {
            float acc = ld(bias, dtype, o);
            for (int64_t i = 0; i < in_features; i++) {
                float prod = ld(x, dtype, b * in_features + i) * ld(weight, dtype, o * in_features + i);
                acc += prod;
            }
            st(out, dtype, b * out_features + o, acc);
        }
    }
    return 0;
}

/* TensorCalc.cpp:221-244 broadcast_source_index for contiguous sources */
static int64_t bcast_index(int64_t out_index, const int64_t* oshape, int orank,
                           const int64_t* sshape, int srank) {
    if (srank == 0) return 0;
    int64_t src = 0, stride = 1, remaining = out_index;
    int off = orank - srank;
    /* strides of the source, innermost first */
    int64_t sstrides[16];
    for (int d = srank - 1; d >= 0; d--) {
        sstrides[d] = stride;
        stride *= sshape[d];
    }
    for (int od = orank - 1; od >= 0; od--) {
        int64_t coord = remaining % oshape[od];
        remaining /= oshape[od];
        int sd = od - off;
        if (sd < 0) continue;
        if (sshape[sd] != 1) src += coord * sstrides[sd];
    }
    return src;
}

/* TensorCalc.cpp:582-663 binary_elementwise + 775-799 add/mul/div */
int oracle_binary(int op, const void* lhs, const int64_t* lshape, int lrank,
                  const void* rhs, const int64_t* rshape, int rrank,
                  void* out, const int64_t* oshape, int orank, int dtype) {
    if (!is_float(dtype)) return fail("binary operands unsupported dtype");
    int64_t n = 1;
    for (int d = 0; d < orank; d++) n *= oshape[d];
    for (int64_t i = 0; i < n; i++) {
        float a = ld(lhs, dtype, bcast_index(i, oshape, orank, lshape, lrank));
        float b = ld(rhs, dtype, bcast_index(i, oshape, orank, rshape, rrank));
        float r;
        switch (op) {
            case 0: r = a + b; break;
            case 1: r = a * b; break;
            case 2: r = a / b; break;
            default: return fail("unknown binary op");
        }
        st(out, dtype, i, r);
    }
    return 0;
}

/* TensorCalc.cpp:562-580 unary_elementwise + relu/sqrt/tanh (775-799) */
int oracle_unary(int op, const void* x, void* out, int dtype, int64_t n) {
    if (!is_float(dtype)) return fail("unary input unsupported dtype");
    for (int64_t i = 0; i < n; i++) {
        float v = ld(x, dtype, i), r;
        switch (op) {
            case 10: r = v > 0.0f ? v : 0.0f; break;
            case 11: r = sqrtf(v); break;
            case 12: r = tanhf(v); break;
            default: return fail("unknown unary op");
        }
        st(out, dtype, i, r);
    }
    return 0;
}

/* Per-node semantics of a fused group: CudaElementwiseKernels.cu:117-159
 * (apply_scalar) and 161-185 (elementwise_kernel): every scalar is an fp32
 * register, Load converts the input element to fp32, Cast passes through,
 * the result is stored once in the output dtype. */
int oracle_elementwise_dag(const OracleScalarNode* nodes, int32_t node_count, uint32_t result,
                           const void* const* inputs, const int32_t* input_dtypes,
                           const int64_t* input_numels, const int32_t* broadcast,
                           int32_t input_count, void* out, int out_dtype, int64_t numel) {
    if (node_count > 32) return fail("elementwise scalar count exceeds kernel max scalars");
    if (result >= 32) return fail("elementwise result scalar id exceeds kernel max scalars");
    for (int i = 0; i < node_count; i++) {
        if (nodes[i].id >= 32) return fail("elementwise scalar id exceeds kernel max scalars");
        if (nodes[i].op == OR_SC_LOAD && (int32_t)nodes[i].input_index >= input_count)
            return fail("elementwise scalar load references invalid input");
    }
    float vals[32];
    for (int64_t lin = 0; lin < numel; lin++) {
        for (int i = 0; i < node_count; i++) {
            const OracleScalarNode* nd = &nodes[i];
            float a = nd->operand_count > 0 ? vals[nd->operands[0]] : 0.0f;
            float b = nd->operand_count > 1 ? vals[nd->operands[1]] : 0.0f;
            float r = 0.0f;
            switch (nd->op) {
                case OR_SC_LOAD: {
                    int ii = (int)nd->input_index;
                    int64_t idx = lin;
                    if (broadcast[ii]) idx = input_numels[ii] == 0 ? 0 : lin % input_numels[ii];
                    r = ld(inputs[ii], input_dtypes[ii], idx);
                    break;
                }
                case OR_SC_CONST: r = (float)nd->constant; break;
                case OR_SC_ADD: r = a + b; break;
                case OR_SC_SUB: r = a - b; break;
                case OR_SC_MUL: r = a * b; break;
                case OR_SC_DIV: r = a / b; break;
                case OR_SC_MAX: r = fmaxf(a, b); break;
                case OR_SC_MIN: r = fminf(a, b); break;
                case OR_SC_NEG: r = -a; break;
                case OR_SC_SQRT: r = sqrtf(a); break;
                case OR_SC_RSQRT: r = 1.0f / sqrtf(a); break;
                case OR_SC_EXP: r = expf(a); break;
                case OR_SC_LOG: r = logf(a); break;
                case OR_SC_TANH: r = tanhf(a); break;
                case OR_SC_RELU: r = fmaxf(a, 0.0f); break;
                case OR_SC_CAST: r = a; break;
                default: return fail("elementwise unknown scalar op");
            }
            vals[nd->id] = r;
        }
        st(out, out_dtype, lin, vals[result]);
    }
    return 0;
}

/* CpuDevice.cpp:611-676 read(DevicePagedTensorView): dense[prefix, grow, :] =
 * page[page_ids[grow / page_size]][prefix, grow % page_size, :] */
int oracle_paged_to_dense(const void* pool, int64_t page_elements, const int32_t* page_ids,
                          int64_t page_count, int64_t prefix, int64_t grow_length,
                          int64_t page_size, int64_t inner, int64_t elem_size, void* out) {
    const uint8_t* src = (const uint8_t*)pool;
    uint8_t* dst = (uint8_t*)out;
    for (int64_t p = 0; p < prefix; p++) {
        for (int64_t g = 0; g < grow_length; g++) {
            int64_t ord = g / page_size, in_page = g % page_size;
            if (ord >= page_count) return fail("paged tensor missing backing page");
            int64_t page = page_ids[ord];
            int64_t s = page * page_elements + (p * page_size + in_page) * inner;
            int64_t d = (p * grow_length + g) * inner;
            memcpy(dst + d * elem_size, src + s * elem_size, (size_t)(inner * elem_size));
        }
    }
    return 0;
}
