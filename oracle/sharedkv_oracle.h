/*
 * CPU restatement of the reference's shared-KV INT8 (C8) path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * product path and the CPU baseline leg of bench.py.  Nothing in the product
 * package may link, load or call it.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the reference checkout, package npu_sparse_attn_sharedkv_int8/).
 */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SKO_DIM 512

/* Exponential shared bit-for-bit with the HIP kernels (Cody-Waite reduction,
 * degree-8 Taylor polynomial in Horner form with explicit fma).  Inputs below
 * -87 return 0 (no subnormal results on either side). */
float sko_expf(float x);
void sko_expf_array(const float *x, float *y, int64_t n);

/* reference.py:47-50  inverse_scale = fp32(1 / fp64(scale)). */
void sko_inverse_scale(const float *scale, float *inverse, int64_t count);

/* reference.py:52-53  code = clamp(round_half_even(fp32(x) * inverse), -127, 127). */
void sko_quantize_f32(const float *x, int64_t rows, const float *inverse, int8_t *out);
void sko_quantize_bf16(const uint16_t *x, int64_t rows, int64_t row_stride,
                       const float *inverse, int8_t *out);

/* cache.py:16-69 + cache_write.cpp:38-73: fused quantize + slot scatter.
 * Slots are int32/int64, flat [T] (page = s / page_size, offset = s % page_size)
 * or paired [T,2] = (page, offset); negative first element, page >= pages or
 * offset outside [0, page_size) skip the row.  Strides are in elements.
 * Returns the number of rows written. */
int64_t sko_cache_write(int8_t *cache, int64_t pages, int64_t page_size, int64_t page_stride,
                        const uint16_t *updates, int64_t tokens, int64_t update_stride,
                        const void *slots, int int64_slots, int paired,
                        int64_t slot_stride, int64_t slot_column_stride,
                        const float *inverse);

/* Input container: reference.py:59-73 (SharedKVCase), with raw pointers.
 * Caches are INT8 [pages][block][1][512] with a page stride in bytes. */
typedef struct {
    const uint16_t *q;              /* BF16 bits [tokens][heads][512] */
    const int8_t *ori;              /* original cache base */
    int64_t ori_stride;             /* bytes between pages */
    const int32_t *ori_table;       /* [batch][ori_table_width] */
    int32_t ori_table_width;
    const int8_t *cmp;              /* compressed cache base (ratio != 1) */
    int64_t cmp_stride;
    const int32_t *cmp_table;
    int32_t cmp_table_width;
    const int32_t *cmp_indices;     /* [tokens][1][topk] for ratio 4 */
    int32_t topk;
    const int32_t *cu_q;            /* [batch + 1] */
    const int32_t *seq_lens;        /* [batch] */
    int32_t batch;
    const float *sink;              /* [heads] */
    const float *ori_scale;         /* [512] */
    const float *cmp_scale;         /* [512] */
    int32_t tokens, heads, block, ratio, window;
    float softmax_scale;
    /* reference.py:73 ori_indices: explicit physical original slots
     * [tokens][1][ori_topk] (page = slot / block, row = slot % block, no
     * block table) replacing the window; NULL for the window. */
    const int32_t *ori_slots;
    int32_t ori_topk;
    int32_t ori_pages;              /* slots at or past ori_pages * block are holes */
} sko_case;

/* Tiling parameters of reference.py:210-212 that fix the numerics. */
typedef struct {
    int32_t tile;              /* keys per tile; a power of two (sum tree) */
    int32_t splits;            /* KV partitions; tile k goes to part k % splits */
    int32_t joint_dense;       /* reference.py:254 joint C128 row */
    int32_t joint_sparse;      /* reference.py:246,254 joint C4 row with log multiplicity */
    int32_t joint_tile_limit;  /* reference.py:212 default 256 */
    int32_t dense_c4;          /* reference.py:246 C4 as multiplicity-weighted dense list */
    int32_t query_group;       /* reference.py:229-231: queries sharing one window/list (>= 1) */
} sko_plan;

/* Optional per-token dumps (heads must be 8).  Any pointer may be NULL.
 *   qcodes [tokens][2 kinds][16][512] int8: rows 0-7 q8 per head, 8-15 q residual
 *   alpha  [tokens][2][8] f32
 *   scores [tokens][128 + cmp_capacity][16] int32: S_hi heads 0-7, S_lo 8-15;
 *          kind-0 list position i at i, kind-1 list position j at 128 + j
 *   probs  [tokens][128 + cmp_capacity][16] int8: p8 heads 0-7, p_low 8-15
 *   values [tokens][tile_capacity][16][512] int32: V_hi rows 0-7, V_lo 8-15,
 *          tiles numbered continuously across kinds
 *   weight_args [tokens][128 + cmp_capacity][8] f32: the argument of each
 *          softmax-weight exponential, logit - running max (reference.py:305),
 *          per list position and head; masked positions included
 * Joint rows (reference.py:175-207) fill qcodes/alpha/scores/probs only. */
typedef struct {
    int8_t *qcodes;
    float *alpha;
    int32_t *scores;
    int8_t *probs;
    int32_t *values;
    int32_t cmp_capacity;
    int32_t tile_capacity;
    float *weight_args;
} sko_debug;

/* reference.py:210-323 tiled_quantized_reference (any query_group; explicit
 * original slots need query_group 1; no row factors; debug dumps need
 * query_group 1).  out: BF16 bits [tokens][heads][512]
 * for tokens < cu_q[batch]; lse: FP32 [tokens][heads] or NULL.  Returns 0 on
 * success, a negative code on invalid arguments. */
int sko_tiled_attention(const sko_case *c, const sko_plan *plan, uint16_t *out, float *lse,
                        sko_debug *debug, int threads);

/* reference.py:175-207 joint_quantized_row on already gathered INT8 rows.
 * kinds = 1 or 2; bias (may be NULL) is added to kind-1 logits. */
void sko_joint_row(const uint16_t *q, int heads, const int8_t *const *rows, const int32_t *counts,
                   const float *const *scales, int kinds, const float *bias, const float *sink,
                   float softmax_scale, uint16_t *out, float *lse);

/* The pairwise (tree) sum both sides use for the tile's softmax weights. */
float sko_tree_sum(const float *x, int32_t count, int32_t padded);

uint16_t sko_f32_to_bf16(float x);
float sko_bf16_to_f32(uint16_t x);

#ifdef __cplusplus
}
#endif
