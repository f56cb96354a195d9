/*
 * C ABI of the MI355X (gfx950) shared-KV INT8 ("C8") attention and INT8 KV
 * cache writer: libsharedkv_hip.so.
 *
 * Plain pointers and sizes only.  Pointer fields hold device addresses; the
 * stream argument is a hipStream_t passed as void*.  Every entry point
 * returns a hipError_t value (0 = success; hipErrorInvalidValue = 1 for a
 * rejected argument block) and launches asynchronously on that stream.
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   SharedKVArgs                      csrc/kernels/c8/args.h:7-14 (200 bytes, same order)
 *   CacheWriteArgs                    csrc/kernels/cache_write.h:4-8 (same order)
 *   launch_sharedkv_c8_sparse         csrc/kernels/c8/c4.cpp:70-71
 *   launch_sharedkv_c8_dense          csrc/kernels/c8/c128.cpp:107-108
 *   launch_sharedkv_c8_sparse_small   csrc/kernels/c8/c4_small.cpp:21-22
 *   launch_cache_write                csrc/kernels/cache_write.cpp:71-80
 * The reference launchers return void; these return the launch status.
 */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Attention arguments (csrc/kernels/c8/args.h:7-14).  Strides are bytes
 * between pages; tables address pages.  Fields this implementation reads:
 *   q (BF16 [tokens][heads][512], heads 1..128), ori/cmp (INT8 pages
 *   [*, 32, 1, 512]), oriScale/cmpScale (FP32 [512]), oriTable/cmpTable
 *   (INT32 [batch][width]), indices (INT32 [tokens][1][topk], ratio 4), cuQ
 *   (INT32 [batch+1]), seqLens (INT32 [batch]), sinks (FP32 [heads]), out
 *   (BF16 [tokens][heads][512]), lse (FP32 [tokens][heads] or 0), partial
 *   (FP32 [rows][splits][8][520] partition states when splits > 1; with
 *   one partition 0, or the re-plan room of sharedkv_c8_partial_bytes),
 *   splits (KV partitions), oriPages (pool size
 *   of the window cache; rows on pages past it are masked), workspace (one
 *   uint32 merge ticket per row, sharedkv_c8_workspace_bytes; zero before the
 *   first launch, and each launch leaves it zero, so launches that may
 *   overlap need their own).  A row is one query token's group of eight
 *   heads: rows = tokens * ceil(heads / 8).  Above eight heads the Q and P
 *   residual codes are off (reference.py:221-222).
 * oriIndices (INT32 [tokens][1][oriTopk], oriTopk <= 1024, or 0): explicit
 * physical original slots (page = slot / 32, row = slot % 32, no table)
 * replacing the window; entries outside [0, oriPages * 32) are masked in
 * place (reference.py:236-239, sparse_gather.h:22-78). */
typedef struct SharedKVArgs {
    uint64_t q, ori, cmp, oriScale, cmpScale, oriTable, cmpTable, indices;
    uint64_t cuQ, seqLens, sinks, out, workspace, lse;
    uint64_t oriStride, cmpStride, partial, oriIndices;
    uint32_t tokens, heads, batch, oriBlock, cmpBlock, oriTableWidth, cmpTableWidth;
    uint32_t ratio, window, topk, splits, oriTopk, oriPages;
    float softmaxScale;
} SharedKVArgs;

/* Cache-writer arguments (csrc/kernels/cache_write.h:4-8).  Strides are in
 * elements: pageStride in INT8 elements, updateStride in BF16 elements,
 * slotStride / slotColumnStride in slot elements. */
typedef struct CacheWriteArgs {
    uint64_t cache, updates, slots, inverseScale;
    uint64_t pageStride, updateStride, slotStride, slotColumnStride;
    uint32_t tokens, pages, pageSize, int64Slots, pairedSlots;
} CacheWriteArgs;

/* Keys per tile of the attention kernels.  Together with SharedKVArgs.splits
 * it fixes the numerics: tile k of a query (kinds in order: original window,
 * then compressed rows) is folded into partition k % splits. */
#define SHAREDKV_C8_TILE 128

/* Optional integer dumps for parity tests (all device pointers, may be 0).
 * Layout per token t, positions P = 128 + cmpCapacity:
 *   qcodes [t][2 kinds][16][512] INT8: rows 0-7 Q head codes, 8-15 residuals
 *   alpha  [t][2][8] FP32
 *   scores [t][P][16] INT32: QK S_hi heads 0-7, S_lo 8-15 per list position
 *          (original window at 0.., compressed list at 128..)
 *   probs  [t][P][16] INT8: p8 heads 0-7, p_low 8-15
 *   values [t][tileCapacity][16][512] INT32: PV V_hi rows 0-7, V_lo 8-15 */
typedef struct SharedKVDebug {
    uint64_t qcodes, alpha, scores, probs, values;
    uint32_t cmpCapacity, tileCapacity;
} SharedKVDebug;

/* C4 attention: SWA128 window plus top-k compressed rows (topk <= 1024).
 * Replaces launch_sharedkv_c8_sparse (c4.cpp:70-71).  `blocks` is accepted
 * for ABI compatibility; 0 launches nothing.  The grid is rows * splits
 * work-groups rounded up to a multiple of 8, rows = tokens * ceil(heads / 8)
 * (plus a rows-wide merge grid in merge mode 1); a launch whose grid would
 * pass 2^31 - 8 work-groups is rejected with hipErrorInvalidValue. */
int launch_sharedkv_c8_sparse(uint32_t blocks, void *stream, const SharedKVArgs *args);

/* Small-capacity C4 entry (c4_small.cpp:21-22), for launches of fewer than
 * 24 query tokens.  The same kernels, except that they also carry the joint
 * route (reference.py:246-267 with joint_sparse) and take it when every live
 * row is short (longest live sequence / 4 <= 128), whatever the block
 * table's width, as the reference's small entry chooses its narrow route
 * from live lengths (c4_small.cpp:10-19).  Through launch_sharedkv_c8_sparse
 * only launches whose compressed block table names at most 128 rows per
 * sequence take it (compiled in, the route costs tiled launches ~1 %). */
int launch_sharedkv_c8_sparse_small(uint32_t blocks, void *stream, const SharedKVArgs *args);

/* C128 attention: SWA128 window plus every compressed row (c128.cpp:107-108).
 * Also serves ratio 1 (window only; the reference's legacy R1 plan). */
int launch_sharedkv_c8_dense(uint32_t blocks, void *stream, const SharedKVArgs *args);

/* Query-grouped attention: the reference device's paired plan (c128.cpp:17-23,
 * numerics reference.py:224-323 with query_group 2, tile_size 256), here
 * chosen by the caller (PreparedAttention(query_group=2)); the reference's
 * launcher picks it inside launch_sharedkv_c8_dense (C128), its operator
 * through launch_sharedkv_paired[_sparse] (attention.py:189-190).  Tokens
 * 2j and 2j + 1 of each request form a group sharing one window list (up to
 * 129 rows) and one compressed list (C128: rows below (p_last + 1) / 128;
 * C4: every row below (p_last + 1) / 4, each token weighing a row by its
 * multiplicity among its own valid top-k entries), each masking what it may
 * not see; 256-key tiles, tile k on partition k % splits (the reference's
 * operator runs one partition), no joint rows.  Any ratio, heads <= 8, no
 * explicit original slots (else hipErrorInvalidValue).  Scratch as for the
 * other launches at rows = tokens; graph padding rows are zero-filled and
 * the launch keeps its partition plan. */
int launch_sharedkv_c8_dense_paired(uint32_t blocks, void *stream, const SharedKVArgs *args);

/* Query-grouped attention in groups of four: the reference device's packed
 * plan (c128.cpp:24-27, numerics reference.py:224-323 with query_group 4,
 * tile_size 256; the operator's launch_sharedkv_packed[_sparse],
 * attention.py:186), chosen by the caller (PreparedAttention(query_group=4)).
 * Tokens 4j .. 4j + 3 of each request form a group sharing one window list
 * (up to 131 rows) and one compressed list; otherwise as
 * launch_sharedkv_c8_dense_paired (same limits, scratch and padding
 * behaviour). */
int launch_sharedkv_c8_dense_packed(uint32_t blocks, void *stream, const SharedKVArgs *args);

/* The same two grouped plans on 128-key tiles (reference.py:224-323 with
 * tile_size 128 and that query_group; no counterpart among the reference's
 * device entries, whose grouped plans are 256-key only), chosen by
 * PreparedAttention(query_group=2 or 4, tile_size=128).  Same limits,
 * scratch and padding behaviour. */
int launch_sharedkv_c8_dense_paired_narrow(uint32_t blocks, void *stream, const SharedKVArgs *args);
int launch_sharedkv_c8_dense_packed_narrow(uint32_t blocks, void *stream, const SharedKVArgs *args);

/* Same launch as launch_sharedkv_c8_sparse / _dense (ratio taken from
 * args->ratio; ungrouped plan), with the integer dumps written to `debug`.
 * Test entry; slower. */
int sharedkv_c8_attention_debug(void *stream, const SharedKVArgs *args, const SharedKVDebug *debug);

/* Fused INT8 quantise + slot scatter (cache_write.cpp:71-80).  `blocks` is
 * accepted for ABI compatibility; 0 launches nothing.  slotStride and
 * slotColumnStride must fit 32 bits (else hipErrorInvalidValue). */
int launch_cache_write(uint32_t blocks, void *stream, const CacheWriteArgs *args);

/* Scratch sizes in bytes for a launch with `rows` = tokens * ceil(heads / 8)
 * rows (the query token count at eight heads).  partial_bytes(rows, 1) is
 * the partition-state room of a one-partition launch's device re-plan: when
 * such a launch (merge mode 0) supplies non-zero `workspace` and `partial`
 * of these sizes, graph padding that leaves fewer live rows than `rows`
 * re-plans the live rows into several partitions merged in the launch, as
 * launches with splits > 1 do (the reference device likewise plans splits
 * from live rows, c4_wide.h:16-41); with partial = 0 it keeps one partition
 * per row.  At most 256 row partitions: min(rows, 256) * 16640 bytes. */
uint64_t sharedkv_c8_workspace_bytes(uint32_t rows, uint32_t splits);
uint64_t sharedkv_c8_partial_bytes(uint32_t rows, uint32_t splits);

/* Allocation-free attention launch.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * launch as the entry the package routes it to: launch_sharedkv_c8_dense
 * (ratio 1 or 128), launch_sharedkv_c8_sparse_small (ratio 4, fewer than 24
 * tokens) or launch_sharedkv_c8_sparse (other ratio-4 launches);
 * args->workspace and args->partial are ignored: the merge tickets and
 * partition states live in a library-owned array of
 * sharedkv_c8_noalloc_scratch_bytes() (16 MiB) per GPU, located on the first
 * call on each device (the stream's device must be current).  The array's
 * layout is fixed: tickets in its first 4096 bytes (1024 rows), partition
 * states from byte 4096 on, so launches of any sizes in any order never
 * find another launch's states where their tickets are.  One-partition
 * launches use the regions only for their device re-plan of a padded
 * launch (at most 256 rows' tickets and states); a launch with splits > 1 whose
 * partial_bytes(rows, splits) exceeds the state region (16 MiB - 4 KiB: 504
 * rows at two partitions) is rejected with hipErrorInvalidValue.  The
 * function calls no hipMalloc or hipFree.  Every call on one GPU uses that
 * GPU's array: calls that may overlap on one GPU (other streams, other
 * threads) race on it. */
int launch_sharedkv_c8_noalloc(uint32_t blocks, void *stream, const SharedKVArgs *args);
uint64_t sharedkv_c8_noalloc_scratch_bytes(void);

/* Byte offsets of the tickets and the partition states that
 * launch_sharedkv_c8_noalloc uses for a launch of `rows` rows and `splits`
 * partitions.  Host-only query (no device call).  Returns 0, or
 * hipErrorInvalidValue when that launch would be rejected. */
int sharedkv_c8_noalloc_layout(uint32_t rows, uint32_t splits, uint64_t *tickets_offset, uint64_t *states_offset);

/* Partition merge placement for launches with splits > 1 (process-wide).
 * Mode 0 (default): fused; the last partition of a query row to finish
 * (ticket in `workspace`) folds the row inside the attention launch.
 * Mode 1: a separate merge kernel follows on the same stream.  Both give
 * identical results.  Returns 0, or hipErrorInvalidValue for other modes. */
int sharedkv_c8_set_merge_mode(int mode);

/* XCD-local partition-state exchange of the fused merge (process-wide; no
 * counterpart in the reference, whose merge runs on one core's memory).
 * Enabled (1, default): on a device where a one-time dispatch probe shows
 * that work-groups whose blockIdx agree modulo 8 run on one XCD, rows whose
 * partitions all run on one XCD pass their states through that XCD's L2;
 * other rows, and every row on other devices, use device-coherent stores
 * and loads.  The probe (first eager launch per device through the launch
 * entries above, never during stream capture or from the allocation-free
 * entry) launches one small kernel and synchronizes the stream once.
 * Disabled (0): device-coherent exchange everywhere.  Results are identical
 * either way.  Returns 0, or hipErrorInvalidValue for other values. */
int sharedkv_c8_set_xcd_local(int enable);

/* The current device's probe result: 1 XCD-local exchange in use, 0 not
 * (probe failed), -1 not probed yet. */
int sharedkv_c8_xcd_local(void);

/* sizeof(SharedKVArgs), sizeof(CacheWriteArgs), library ABI version. */
uint32_t sharedkv_attention_args_size(void);
uint32_t sharedkv_cache_args_size(void);
uint32_t sharedkv_abi_version(void);

#ifdef __cplusplus
}
#endif
