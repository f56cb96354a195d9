/*
 * CPU restatement of the reference's shared-KV INT8 (C8) attention and its
 * INT8 cache writer.  TEST INFRASTRUCTURE ONLY: the parity checker for the HIP
 * kernels and the CPU-baseline leg of bench.py; the product never links it.
 *
 * Reference files (relative to the reference checkout):
 *   npu_sparse_attn_sharedkv_int8/reference.py   algorithm (cited per function)
 *   csrc/kernels/cache_write.cpp:38-73           writer slot decoding and skips
 *
 * Floating-point contract.  Every FP32 operation below is an IEEE basic
 * operation in the order reference.py performs it (compile with
 * -ffp-contract=off, no fast-math).  Two choices are ours, not torch's:
 *   - exp is sko_expf (Cody-Waite + Taylor), identical to the HIP kernels';
 *     torch.exp differs from it by at most an ulp on rare inputs;
 *   - the per-tile sum of softmax weights (reference.py:306 weights.sum(-1))
 *     is a pairwise tree over the tile's positions, and a joint row's sum
 *     (reference.py:196) one such tree per kind, added in kind order;
 *     torch's order is its own.
 * Both are pinned against vectors generated from reference.py (tests/golden).
 */
#include "sharedkv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define D SKO_DIM
#define C127 ((float)(1.0 / 127.0))
#define MASKED (-1e30f)

/* ------------------------------------------------------------------ */
/* Scalar helpers                                                       */
/* ------------------------------------------------------------------ */

/* exp(x) by Cody & Waite argument reduction x = n*ln2 + r, |r| <= ln2/2, with
 * ln2 split into a 16-bit head and a tail, and the Taylor series of e^r to
 * degree 8 evaluated in Horner form with fused multiply-adds.  Truncation
 * error is below 3e-10 relative on the reduced range. */
float sko_expf(float x)
{
    if (!(x >= -87.0f)) return x != x ? x : 0.0f;
    if (x > 88.0f) return INFINITY;
    const float log2e = 1.44269504088896341f;
    const float ln2_hi = 0.693145751953125f;          /* ln 2 rounded to 16 bits */
    const float ln2_lo = 1.42860682030941723212e-6f;  /* ln 2 - ln2_hi */
    float n = rintf(x * log2e);
    float r = fmaf(-n, ln2_hi, x);
    r = fmaf(-n, ln2_lo, r);
    float p = 1.0f / 40320.0f;
    p = fmaf(p, r, 1.0f / 5040.0f);
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

void sko_expf_array(const float *x, float *y, int64_t n)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = sko_expf(x[i]);
}

uint16_t sko_f32_to_bf16(float x)
{
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float sko_bf16_to_f32(uint16_t x)
{
    uint32_t u = (uint32_t)x << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* log of a multiplicity count (reference.py:249, 261 cmp_multiplicity.log()),
 * evaluated in double and rounded once to FP32.  For every count 1..1024
 * the exact ln(k) lies at least 4e-4 FP32 ulp from an FP32 rounding midpoint,
 * so this is the correctly rounded value, equal to glibc logf and torch.log
 * at every count, and any double log accurate to a few ulps gives the same
 * float (the HIP kernel uses the device library's). */
static float log_count(float count)
{
    return (float)log((double)count);
}

/* Pairwise sum: level by level, element 2i plus element 2i+1; the input is
 * zero-padded to `padded` (a power of two >= count). */
float sko_tree_sum(const float *x, int32_t count, int32_t padded)
{
    float buf[1024];
    if (padded < 1) return 0.0f;
    float *v = padded <= 1024 ? buf : (float *)malloc(sizeof(float) * (size_t)padded);
    for (int32_t i = 0; i < padded; ++i) v[i] = i < count ? x[i] : 0.0f;
    for (int32_t width = padded; width > 1; width /= 2)
        for (int32_t i = 0; i < width / 2; ++i) v[i] = v[2 * i] + v[2 * i + 1];
    float s = v[0];
    if (v != buf) free(v);
    return s;
}

static int32_t pow2_at_least(int32_t n)
{
    int32_t p = 1;
    while (p < n) p *= 2;
    return p;
}

/* ------------------------------------------------------------------ */
/* KV encoding and the cache writer                                     */
/* ------------------------------------------------------------------ */

/* reference.py:47-50 */
void sko_inverse_scale(const float *scale, float *inverse, int64_t count)
{
    for (int64_t i = 0; i < count; ++i) inverse[i] = (float)(1.0 / (double)scale[i]);
}

static inline int8_t encode(float x, float inverse)
{
    /* reference.py:53: round half-even, then clamp to [-127, 127]. */
    float v = rintf(x * inverse);
    v = v < -127.0f ? -127.0f : v > 127.0f ? 127.0f : v;
    return (int8_t)v;
}

/* reference.py:52-53 */
void sko_quantize_f32(const float *x, int64_t rows, const float *inverse, int8_t *out)
{
    for (int64_t r = 0; r < rows; ++r)
        for (int c = 0; c < D; ++c) out[r * D + c] = encode(x[r * D + c], inverse[c]);
}

void sko_quantize_bf16(const uint16_t *x, int64_t rows, int64_t row_stride,
                       const float *inverse, int8_t *out)
{
    for (int64_t r = 0; r < rows; ++r)
        for (int c = 0; c < D; ++c) out[r * D + c] = encode(sko_bf16_to_f32(x[r * row_stride + c]), inverse[c]);
}

/* cache.py:16-22 contract; slot decode and skip rules of cache_write.cpp:59-72. */
int64_t sko_cache_write(int8_t *cache, int64_t pages, int64_t page_size, int64_t page_stride,
                        const uint16_t *updates, int64_t tokens, int64_t update_stride,
                        const void *slots, int int64_slots, int paired,
                        int64_t slot_stride, int64_t slot_column_stride,
                        const float *inverse)
{
    int64_t written = 0;
    for (int64_t row = 0; row < tokens; ++row) {
        int64_t first = int64_slots ? ((const int64_t *)slots)[row * slot_stride]
                                    : ((const int32_t *)slots)[row * slot_stride];
        if (first < 0) continue;
        int64_t page, offset;
        if (paired) {
            page = first;
            offset = int64_slots ? ((const int64_t *)slots)[row * slot_stride + slot_column_stride]
                                 : ((const int32_t *)slots)[row * slot_stride + slot_column_stride];
        } else {
            page = first / page_size;
            offset = first % page_size;
        }
        if (page >= pages || offset < 0 || offset >= page_size) continue;
        int8_t *dst = cache + page * page_stride + offset * D;
        for (int c = 0; c < D; ++c) dst[c] = encode(sko_bf16_to_f32(updates[row * update_stride + c]), inverse[c]);
        ++written;
    }
    return written;
}

/* ------------------------------------------------------------------ */
/* Attention                                                            */
/* ------------------------------------------------------------------ */

/* reference.py:82-85 gather: logical row -> physical page via the block
 * table; without a table (reference.py:88-90 gather_slots) the index is a
 * physical slot. */
static const int8_t *row_address(const int8_t *cache, int64_t stride, const int32_t *table,
                                 int32_t width, int32_t block, int32_t batch, int64_t index)
{
    int64_t page = table ? table[(int64_t)batch * width + index / block] : index / block;
    return cache + page * stride + (index % block) * D;
}

/* reference.py:274-279 (and 183-187): fold the per-channel scale into Q and
 * split it into an INT8 head plus an INT8 residual. */
static void encode_query(const uint16_t *q, int heads, const float *scale, float softmax_scale,
                         int32_t *high, int32_t *low, float *alpha, float *logit_scale)
{
    for (int h = 0; h < heads; ++h) {
        float folded[D];
        float amax = 0.0f;
        for (int c = 0; c < D; ++c) {
            folded[c] = sko_bf16_to_f32(q[h * D + c]) * scale[c];
            float a = fabsf(folded[c]);
            amax = a > amax ? a : amax;
        }
        float al = amax * C127;
        al = al < 1e-12f ? 1e-12f : al;
        float inv = 1.0f / al;
        for (int c = 0; c < D; ++c) {
            float n = folded[c] * inv;
            n = n < -127.0f ? -127.0f : n > 127.0f ? 127.0f : n;
            float hi = rintf(n);
            high[h * D + c] = (int32_t)hi;
            low[h * D + c] = (int32_t)rintf((n - hi) * 127.0f);
        }
        alpha[h] = al;
        logit_scale[h] = al * softmax_scale;
    }
}

static inline int32_t dot_i8(const int32_t *a, const int8_t *b)
{
    int32_t s = 0;
    for (int c = 0; c < D; ++c) s += a[c] * (int32_t)b[c];
    return s;
}

typedef struct {
    const int8_t *cache;
    int64_t stride;
    const int32_t *table;
    int32_t width;
    const float *scale;
    int32_t length;          /* list positions */
    int64_t *index;          /* logical row per position */
    uint8_t *valid;
    float *multiplicity;     /* dense_c4 / joint_sparse lists, else NULL */
} kind_list;

/* reference.py:175-207 joint_quantized_row. */
void sko_joint_row(const uint16_t *q, int heads, const int8_t *const *rows, const int32_t *counts,
                   const float *const *scales, int kinds, const float *bias, const float *sink,
                   float softmax_scale, uint16_t *out, float *lse)
{
    int32_t total = 0;
    for (int k = 0; k < kinds; ++k) total += counts[k];
    float *scores = (float *)malloc(sizeof(float) * (size_t)(heads * (total ? total : 1)));
    int32_t *hi = (int32_t *)malloc(sizeof(int32_t) * heads * D);
    int32_t *lo = (int32_t *)malloc(sizeof(int32_t) * heads * D);
    float alpha[128], asc[128];
    int32_t offset = 0;
    for (int k = 0; k < kinds; ++k) {
        encode_query(q, heads, scales[k], softmax_scale, hi, lo, alpha, asc);
        for (int32_t j = 0; j < counts[k]; ++j) {
            const int8_t *row = rows[k] + (int64_t)j * D;
            for (int h = 0; h < heads; ++h) {
                float dot = (float)dot_i8(hi + h * D, row) + (float)dot_i8(lo + h * D, row) * C127;
                float logit = dot * asc[h];
                if (k == 1 && bias) logit = logit + bias[j];
                scores[h * total + offset + j] = logit;
            }
        }
        offset += counts[k];
    }
    float *w = (float *)malloc(sizeof(float) * (size_t)(total ? total : 1));
    for (int h = 0; h < heads; ++h) {
        float m = sink[h];
        for (int32_t j = 0; j < total; ++j) m = scores[h * total + j] > m ? scores[h * total + j] : m;
        for (int32_t j = 0; j < total; ++j) w[j] = sko_expf(scores[h * total + j] - m);
        /* weights.sum(-1) over the concatenated kinds (reference.py:196): a
         * pairwise tree per kind, the kinds' sums added in order. */
        float wsum = 0.0f;
        offset = 0;
        for (int k = 0; k < kinds; ++k) {
            const float part = sko_tree_sum(w + offset, counts[k], pow2_at_least(counts[k] ? counts[k] : 1));
            wsum = k ? wsum + part : part;
            offset += counts[k];
        }
        float den = sko_expf(sink[h] - m) + wsum;
        float acc[D];
        for (int c = 0; c < D; ++c) acc[c] = 0.0f;
        offset = 0;
        for (int k = 0; k < kinds; ++k) {
            float sc[D];
            for (int c = 0; c < D; ++c) sc[c] = scales[k][c] * C127;
            int32_t vh[D], vl[D];
            memset(vh, 0, sizeof vh);
            memset(vl, 0, sizeof vl);
            for (int32_t j = 0; j < counts[k]; ++j) {
                float x = w[offset + j] * 127.0f;
                float ph = rintf(x);
                int32_t p8 = (int32_t)ph, pl = (int32_t)rintf((x - ph) * 127.0f);
                const int8_t *row = rows[k] + (int64_t)j * D;
                for (int c = 0; c < D; ++c) {
                    vh[c] += p8 * row[c];
                    vl[c] += pl * row[c];
                }
            }
            for (int c = 0; c < D; ++c) {
                float dot = (float)vh[c] + (float)vl[c] * C127;
                acc[c] = acc[c] + dot * sc[c];
            }
            offset += counts[k];
        }
        for (int c = 0; c < D; ++c) out[h * D + c] = sko_f32_to_bf16(acc[c] / den);
        if (lse) lse[h] = m + logf(den);
    }
    free(w);
    free(scores);
    free(hi);
    free(lo);
}

/* One query row of reference.py:224-323.  Queries of one request form
 * groups of pl->query_group consecutive tokens (reference.py:229-231); a
 * group shares one window list and one compressed list, each query masking
 * what it may not see. */
static void attend_token(const sko_case *c, const sko_plan *pl, int32_t b, int32_t t, int32_t last,
                         uint16_t *out, float *lse, sko_debug *dbg)
{
    const int H = c->heads;
    const int32_t length = c->seq_lens[b];
    const int64_t position = (int64_t)length - last + t;
    const int residual = H <= 8;   /* reference.py:221-222 */
    const int32_t G = pl->query_group;
    const int32_t first_q = c->cu_q[b];
    const int32_t group_first = first_q + (t - first_q) / G * G;
    const int32_t group_last = (last < group_first + G ? last : group_first + G) - 1;
    const int64_t first_pos = (int64_t)length - last + group_first;
    const int64_t last_pos = (int64_t)length - last + group_last;
    kind_list lists[2];
    int kinds = 1;

    /* Kind 0: SWA window, reference.py:232-234 (the group's positions
     * max(0, first_pos + 1 - window) .. last_pos, valid where they fall in
     * this query's own window), or the explicit physical slots of
     * reference.py:236-239 (every entry keeps its place; entries outside
     * [0, pages * block) are holes). */
    int64_t first = first_pos + 1 - c->window;
    if (first < 0) first = 0;
    int64_t own_first = position + 1 - c->window;
    if (own_first < 0) own_first = 0;
    int32_t ori_count = c->ori_slots ? c->ori_topk : (int32_t)(last_pos + 1 - first);
    lists[0] = (kind_list){c->ori, c->ori_stride, c->ori_slots ? NULL : c->ori_table, c->ori_table_width,
                           c->ori_scale, ori_count, malloc(sizeof(int64_t) * (ori_count ? ori_count : 1)),
                           malloc(ori_count ? ori_count : 1), NULL};
    for (int32_t i = 0; i < ori_count; ++i) {
        if (c->ori_slots) {
            int64_t slot = c->ori_slots[(int64_t)t * c->ori_topk + i];
            lists[0].index[i] = slot;
            lists[0].valid[i] = slot >= 0 && slot < (int64_t)c->ori_pages * c->block;
        } else {
            lists[0].index[i] = first + i;
            lists[0].valid[i] = first + i >= own_first && first + i <= position;
        }
    }

    /* Kind 1: compressed rows, reference.py:242-253.  C128 lists the
     * group's rows, valid below this query's own count. */
    if (c->ratio != 1) {
        kinds = 2;
        int64_t count = (position + 1) / c->ratio;
        int64_t group_count = (last_pos + 1) / c->ratio;
        int32_t n = c->ratio == 4 ? c->topk : (int32_t)group_count;
        kind_list *k = &lists[1];
        *k = (kind_list){c->cmp, c->cmp_stride, c->cmp_table, c->cmp_table_width, c->cmp_scale,
                         n, malloc(sizeof(int64_t) * (n ? n : 1)), malloc(n ? n : 1), NULL};
        for (int32_t j = 0; j < n; ++j) {
            int64_t idx = c->ratio == 4 ? c->cmp_indices[(int64_t)t * c->topk + j] : j;
            k->index[j] = idx;
            k->valid[j] = idx >= 0 && idx < count;
        }
        if (c->ratio == 4 && (G > 1 || pl->dense_c4 || pl->joint_sparse)) {
            /* reference.py:246-249: multiplicity over arange of the group's
             * compressed rows (every valid index lies below it). */
            float *mult = calloc(group_count ? group_count : 1, sizeof(float));
            for (int32_t j = 0; j < n; ++j)
                if (k->valid[j]) mult[k->index[j]] += 1.0f;
            free(k->index);
            free(k->valid);
            k->length = (int32_t)group_count;
            k->index = malloc(sizeof(int64_t) * (group_count ? group_count : 1));
            k->valid = malloc(group_count ? group_count : 1);
            for (int64_t j = 0; j < group_count; ++j) {
                k->index[j] = j;
                k->valid[j] = mult[j] > 0.0f;
            }
            k->multiplicity = mult;
        } else if (c->ratio == 4 && count < n && n <= 1024) {
            /* reference.py:250-252: compact valid indices in order. */
            int32_t m = 0;
            for (int32_t j = 0; j < n; ++j)
                if (k->valid[j]) k->index[m++] = k->index[j];
            for (int32_t j = 0; j < m; ++j) k->valid[j] = 1;
            k->length = m;
        }
    }

    const int32_t N = pl->tile, S = pl->splits;
    uint16_t *orow = out + (int64_t)t * H * D;
    float *lrow = lse ? lse + (int64_t)t * H : NULL;

    /* Joint row, reference.py:254-267. */
    if (((pl->joint_dense && c->ratio == 128) || (pl->joint_sparse && c->ratio == 4)) && S == 1
        && (c->ratio == 128 || G == 1) && N <= pl->joint_tile_limit && kinds == 2 && lists[1].length <= N && lists[0].length <= N
        && (pl->joint_sparse || lists[1].length > 0)) {
        const int8_t *rows[2];
        int32_t counts[2];
        float *bias = NULL;
        int8_t *gathered[2];
        for (int k = 0; k < 2; ++k) {
            kind_list *L = &lists[k];
            gathered[k] = malloc((size_t)(L->length ? L->length : 1) * D);
            int32_t m = 0;
            for (int32_t j = 0; j < L->length; ++j) {
                if (!L->valid[j]) continue;
                memcpy(gathered[k] + (int64_t)m * D,
                       row_address(L->cache, L->stride, L->table, L->width, c->block, b, L->index[j]), D);
                ++m;
            }
            rows[k] = gathered[k];
            counts[k] = m;
        }
        if (pl->joint_sparse && c->ratio == 4) {
            bias = malloc(sizeof(float) * (counts[1] ? counts[1] : 1));
            int32_t m = 0;
            for (int32_t j = 0; j < lists[1].length; ++j)
                if (lists[1].valid[j]) bias[m++] = log_count(lists[1].multiplicity[j]);
        }
        const float *scales[2] = {c->ori_scale, c->cmp_scale};
        sko_joint_row(c->q + (int64_t)t * H * D, H, rows, counts, scales, 2, bias, c->sink,
                      c->softmax_scale, orow, lrow);
        if (dbg && H == 8) {
            int32_t *hi = malloc(sizeof(int32_t) * H * D), *lo = malloc(sizeof(int32_t) * H * D);
            float alpha[8], asc[8];
            for (int k = 0; k < 2; ++k) {
                encode_query(c->q + (int64_t)t * H * D, H, k ? c->cmp_scale : c->ori_scale,
                             c->softmax_scale, hi, lo, alpha, asc);
                if (dbg->qcodes) {
                    int8_t *qc = dbg->qcodes + ((int64_t)t * 2 + k) * 16 * D;
                    for (int h = 0; h < 8; ++h)
                        for (int d = 0; d < D; ++d) {
                            qc[h * D + d] = (int8_t)hi[h * D + d];
                            qc[(8 + h) * D + d] = (int8_t)lo[h * D + d];
                        }
                }
                if (dbg->alpha) memcpy(dbg->alpha + ((int64_t)t * 2 + k) * 8, alpha, sizeof alpha);
            }
            free(hi);
            free(lo);
        }
        for (int k = 0; k < 2; ++k) free(gathered[k]);
        free(bias);
        goto done;
    }

    {
        float *mx = malloc(sizeof(float) * S * H);
        float *den = malloc(sizeof(float) * S * H);
        float *num = calloc((size_t)S * H * D, sizeof(float));
        for (int32_t s = 0; s < S; ++s)
            for (int h = 0; h < H; ++h) {
                mx[s * H + h] = c->sink[h];
                den[s * H + h] = s == 0 ? 1.0f : 0.0f;
            }
        int32_t *qhi = malloc(sizeof(int32_t) * H * D), *qlo = malloc(sizeof(int32_t) * H * D);
        int8_t *kv = malloc((size_t)N * D);
        float *logit = malloc(sizeof(float) * H * N), *w = malloc(sizeof(float) * N);
        int32_t *p8 = malloc(sizeof(int32_t) * H * N), *plo = malloc(sizeof(int32_t) * H * N);
        float alpha[128], asc[128];
        int32_t tile_number = 0;
        const int32_t cap = dbg ? 128 + dbg->cmp_capacity : 0;
        for (int k = 0; k < kinds; ++k) {
            kind_list *L = &lists[k];
            encode_query(c->q + (int64_t)t * H * D, H, L->scale, c->softmax_scale, qhi, qlo, alpha, asc);
            if (!residual) memset(qlo, 0, sizeof(int32_t) * H * D);
            if (dbg && H == 8) {
                if (dbg->qcodes) {
                    int8_t *qc = dbg->qcodes + ((int64_t)t * 2 + k) * 16 * D;
                    for (int h = 0; h < 8; ++h)
                        for (int d = 0; d < D; ++d) {
                            qc[h * D + d] = (int8_t)qhi[h * D + d];
                            qc[(8 + h) * D + d] = (int8_t)qlo[h * D + d];
                        }
                }
                if (dbg->alpha) memcpy(dbg->alpha + ((int64_t)t * 2 + k) * 8, alpha, 8 * sizeof(float));
            }
            for (int32_t start = 0; start < L->length; start += N) {
                const int32_t part = tile_number % S;
                const int32_t tn = tile_number++;
                const int32_t n = L->length - start < N ? L->length - start : N;
                /* reference.py:283-286: masked rows are zero. */
                for (int32_t j = 0; j < n; ++j) {
                    if (L->valid[start + j])
                        memcpy(kv + (int64_t)j * D,
                               row_address(L->cache, L->stride, L->table, L->width, c->block, b,
                                           L->index[start + j]), D);
                    else
                        memset(kv + (int64_t)j * D, 0, D);
                }
                /* reference.py:287-302 */
                for (int h = 0; h < H; ++h)
                    for (int32_t j = 0; j < n; ++j) {
                        int32_t sh = dot_i8(qhi + h * D, kv + (int64_t)j * D);
                        int32_t sl = residual ? dot_i8(qlo + h * D, kv + (int64_t)j * D) : 0;
                        float dots = (float)sh;
                        if (residual) dots = dots + (float)sl * C127;
                        float lg = dots * asc[h];
                        if (k == 1 && L->multiplicity) {
                            float m = L->multiplicity[L->index[start + j]];
                            lg = lg + log_count(m < 1.0f ? 1.0f : m);
                        }
                        if (!L->valid[start + j]) lg = MASKED;
                        logit[h * N + j] = lg;
                        if (dbg && dbg->scores && H == 8) {
                            int32_t *row = dbg->scores + ((int64_t)t * cap + (k ? 128 : 0) + start + j) * 16;
                            row[h] = sh;
                            row[8 + h] = sl;
                        }
                    }
                /* reference.py:303-316 */
                const int32_t padded = pow2_at_least(N);
                for (int h = 0; h < H; ++h) {
                    float *m_old = &mx[part * H + h];
                    float m_new = *m_old;
                    for (int32_t j = 0; j < n; ++j) m_new = logit[h * N + j] > m_new ? logit[h * N + j] : m_new;
                    float factor = sko_expf(*m_old - m_new);
                    for (int32_t j = 0; j < n; ++j) {
                        w[j] = sko_expf(logit[h * N + j] - m_new);
                        if (dbg && dbg->weight_args && H == 8)
                            dbg->weight_args[((int64_t)t * cap + (k ? 128 : 0) + start + j) * 8 + h] =
                                logit[h * N + j] - m_new;
                    }
                    den[part * H + h] = den[part * H + h] * factor + sko_tree_sum(w, n, padded);
                    for (int32_t j = 0; j < n; ++j) {
                        float x = w[j] * 127.0f;
                        float hi = rintf(x);
                        p8[h * N + j] = (int32_t)hi;
                        plo[h * N + j] = residual ? (int32_t)rintf((x - hi) * 127.0f) : 0;
                        if (dbg && dbg->probs && H == 8) {
                            int8_t *row = dbg->probs + ((int64_t)t * cap + (k ? 128 : 0) + start + j) * 16;
                            row[h] = (int8_t)p8[h * N + j];
                            row[8 + h] = (int8_t)plo[h * N + j];
                        }
                    }
                    int32_t vh[D], vl[D];
                    memset(vh, 0, sizeof vh);
                    memset(vl, 0, sizeof vl);
                    for (int32_t j = 0; j < n; ++j) {
                        const int8_t *row = kv + (int64_t)j * D;
                        const int32_t a = p8[h * N + j], bl = plo[h * N + j];
                        for (int d = 0; d < D; ++d) {
                            vh[d] += a * row[d];
                            vl[d] += bl * row[d];
                        }
                    }
                    if (dbg && dbg->values && H == 8 && tn < dbg->tile_capacity) {
                        int32_t *v = dbg->values + ((int64_t)t * dbg->tile_capacity + tn) * 16 * D;
                        memcpy(v + h * D, vh, sizeof vh);
                        memcpy(v + (8 + h) * D, vl, sizeof vl);
                    }
                    float *acc = num + ((int64_t)part * H + h) * D;
                    for (int d = 0; d < D; ++d) {
                        float dots = (float)vh[d];
                        if (residual) dots = dots + (float)vl[d] * C127;
                        float pv = dots * L->scale[d] * C127;
                        acc[d] = acc[d] * factor + pv;
                    }
                    *m_old = m_new;
                }
            }
        }
        /* reference.py:317-323: merge the partitions. */
        for (int h = 0; h < H; ++h) {
            float top = mx[h];
            for (int32_t s = 1; s < S; ++s) top = mx[s * H + h] > top ? mx[s * H + h] : top;
            float dsum = 0.0f;
            float acc[D];
            for (int d = 0; d < D; ++d) acc[d] = 0.0f;
            for (int32_t s = 0; s < S; ++s) {
                float f = sko_expf(mx[s * H + h] - top);
                const float *src = num + ((int64_t)s * H + h) * D;
                for (int d = 0; d < D; ++d) acc[d] = acc[d] + src[d] * f;
                dsum = dsum + den[s * H + h] * f;
            }
            for (int d = 0; d < D; ++d) orow[h * D + d] = sko_f32_to_bf16(acc[d] / dsum);
            if (lrow) lrow[h] = top + logf(dsum);
        }
        free(mx); free(den); free(num); free(qhi); free(qlo); free(kv);
        free(logit); free(w); free(p8); free(plo);
    }
done:
    for (int k = 0; k < kinds; ++k) {
        free(lists[k].index);
        free(lists[k].valid);
        free(lists[k].multiplicity);
    }
}

int sko_tiled_attention(const sko_case *c, const sko_plan *pl, uint16_t *out, float *lse,
                        sko_debug *dbg, int threads)
{
    if (!c || !pl || !out || c->heads <= 0 || c->heads > 128 || c->block <= 0 || c->window <= 0)
        return -1;
    if (c->ratio != 1 && c->ratio != 4 && c->ratio != 128) return -2;
    if (pl->tile <= 0 || (pl->tile & (pl->tile - 1)) || pl->splits <= 0 || pl->query_group <= 0) return -3;
    if (pl->query_group > 1 && (c->ori_slots || dbg)) return -10;   /* reference.py:236-237 */
    /* reference.py:258 asserts residual codes (at most eight heads) for
     * joint rows; refused here for the whole plan. */
    if ((pl->joint_dense || pl->joint_sparse) && c->heads > 8) return -11;
    if (c->ratio != 1 && (!c->cmp || !c->cmp_table || !c->cmp_scale)) return -4;
    if (c->ratio == 4 && (!c->cmp_indices || c->topk <= 0)) return -5;
    if (dbg && (c->window > 128 || (c->ori_slots && c->ori_topk > 128))) return -6;
    if (c->ori_slots && (c->ori_topk <= 0 || c->ori_pages <= 0)) return -9;
    int32_t total = c->cu_q[c->batch];
    if (total > c->tokens) return -7;
    /* Flatten (batch, token) pairs so OpenMP can split tokens evenly. */
    int32_t *owner = malloc(sizeof(int32_t) * (total ? total : 1));
    for (int32_t b = 0; b < c->batch; ++b) {
        if (c->cu_q[b + 1] - c->cu_q[b] > c->seq_lens[b]) {
            free(owner);
            return -8;   /* reference.py:104-105 */
        }
        for (int32_t t = c->cu_q[b]; t < c->cu_q[b + 1]; ++t) owner[t] = b;
    }
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
    for (int32_t t = 0; t < total; ++t) {
        int32_t b = owner[t];
        attend_token(c, pl, b, t, c->cu_q[b + 1], out, lse, dbg);
    }
    free(owner);
    return 0;
}
