// MI355X (gfx950) shared-KV INT8 attention ("C8") and INT8 KV cache writer.
//
// Behaviour follows the reference's p101 C8 path (paths relative to the
// reference checkout):
//   algorithm       npu_sparse_attn_sharedkv_int8/reference.py:210-323
//   selection       csrc/kernels/c8/attention_impl.h:27-92 (window, C4/C128 lists)
//   live metadata   csrc/kernels/c8/attention_impl.h:102-137 (padded graph rows)
//   C4 compaction   csrc/kernels/c8/gather.h:22-55, reference.py:250-252
//   split merge     csrc/kernels/c8/attention_impl.h:397-441, reference.py:317-323
//   cache writer    csrc/kernels/cache_write.cpp:9-88
//
// Design (one GPU, HBM bound).  One work-group of 8 waves (two per SIMD) per
// (query row, KV partition), one work-group per CU; a query row is one token
// and eight of its heads (tokens with more heads take several rows).
// Partition `part` owns tiles part, part + S, ... of the row's key list
// (window rows or explicit original slots, then compressed rows, cut into
// 128-key tiles).
//   prologue   every load of the row that the selection needs (metadata,
//              indices, Q) is issued at once from kernel arguments that the
//              build preloads into SGPRs: one memory round trip, with the
//              argument block read alongside; sinks and scales follow
//   addresses  the partition's rows become page codes (page * 32 + row in
//              page, -1 = masked) and HBM addresses in LDS after one round
//              trip of block-table reads (issued before the C4 compaction
//              scan); the first tile is requested at once, and Q is encoded
//              for both cache kinds while its rows are in flight
//   tiles      rows go from HBM straight into a two-tile LDS ring by LDS DMA
//              (whole 512-byte rows per instruction); the next tile is in
//              flight while the current one is computed.  QK: each wave takes
//              16 keys, v_mfma_i32_16x16x64_i8 with the 16 MFMA rows = 8 heads
//              x {code, residual}; PV: each wave takes 64 output columns and
//              reads V transposed with ds_read_b64_tr_b8
//   softmax    FP32 in registers; max and pairwise sums cross waves in LDS
//   partials   with S > 1 partitions, FP32 [num, max, den] go to `partial`;
//              the last partition of a row to finish (a ticket per row in
//              `workspace`) folds them, or c8_merge does in a second launch
// One-partition C4 and window-only launches of more rows than CUs (prefill,
// large decode batches; any head count, no explicit slots) run c8_rows instead:
// two four-wave work-groups per CU with one tile buffer each, each taking
// rows in turn, so that one row's tile chain fills the other's waits.
// Integer partials are exact, so any assignment of keys to lanes gives the
// reference's integers; the FP32 sequence below is kept in the reference's
// order with contraction disabled.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include "sharedkv_hip.h"

#pragma clang fp contract(off)

namespace {

constexpr int D = 512;
constexpr int HEADS = 8;               // heads per work-group (one MFMA row block with residual rows)
constexpr int MAX_HEADS = 128;
constexpr int N = SHAREDKV_C8_TILE;    // keys per tile
// Partition plan of a launch's live rows (the host's choose_splits rule):
// one partition per tile of the longest row while rows x tiles stay within
// PLAN_ONE_TILE work items and the launch's work items allow it (a row then
// waits for one tile and the merge); else PLAN_FEW partitions while rows x
// PLAN_FEW work-groups fit the PLAN_CUS compute units, else PLAN_MANY.
constexpr int32_t PLAN_CUS = 256, PLAN_FEW = 5, PLAN_MANY = 3, PLAN_ONE_TILE = 112;
constexpr int THREADS = 512;           // 8 waves: two per SIMD
constexpr int WAVES = THREADS / 64;
constexpr int PROW = N + 16;           // LDS row stride of the P codes
constexpr int CODE_TILES = 12;         // tiles whose row codes are resident at once
constexpr int MAX_LIST = 1024;         // C4 top-k capacity of the index list
constexpr int PART_FLOATS = 520;       // per (row, split, head): 512 numerator, max, denominator
constexpr int FOLD_SLOT = 514;         // partition 0, head 0: partitions to fold (merge launch), 0 = none
constexpr int WINDOW = 128;
constexpr int BLOCK_ROWS = 32;
constexpr uint32_t MAX_SPLITS = 16;
// C4 launches of fewer query tokens go through the small-launch entry
// (the reference host's rule, c8_attention.py:111-112 there: tokens < its
// 24 cores).
constexpr uint32_t SMALL_TOKENS = 24;
static_assert(N == 128 && WINDOW == N && WAVES == 8, "one window tile of 128 keys; 8 waves x 16 keys");
static_assert(MAX_LIST == 2 * THREADS, "two C4 index entries per thread");

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v2i lds_v2i;
typedef __attribute__((address_space(3))) int8_t lds_i8;

// Device addresses arrive as integers; view them in the global address space
// so the compiler issues global_load (vector memory counter only), not flat.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T *gptr(uint64_t a)
{
    return reinterpret_cast<const __attribute__((address_space(1))) T *>(a);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits) { return __uint_as_float(bits << 16); }

// Two floats to packed BF16 with one v_cvt_pk_bf16_f32: round to nearest
// even, NaN to the quiet NaN with the upper payload bits kept.  This equals
// torch's .bfloat16() (and the CPU checker's bit-level rounding) for every
// 32-bit input.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// exp(x) for x <= 0 (or NaN), the only arguments the softmax and the merge
// produce (differences x - max(...)): Cody & Waite reduction x = n ln2 + r
// with a 16-bit head of ln2 and its tail, then the degree-8 Taylor series of
// e^r in Horner form with fma, scaled by 2^n; below -87 the result is 0.  The
// CPU checker evaluates the identical sequence (its x > 88 overflow branch
// never fires for such arguments), so the softmax weights and the INT8 P
// codes derived from them agree bit for bit.
__device__ __forceinline__ float sk_expf_nonpos(float x)
{
    // Evaluated without a branch: the series runs on a clamped argument and
    // the result is selected, which keeps both exponentials of a lane in one
    // instruction stream.
    const bool in_range = x >= -87.0f;
    const float xr = in_range ? x : -87.0f;
    float n = __builtin_rintf(xr * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, xr);
    r = __builtin_fmaf(-n, 1.42860682030941723212e-6f, r);
    float p = 1.0f / 40320.0f;
    p = __builtin_fmaf(p, r, 1.0f / 5040.0f);
    p = __builtin_fmaf(p, r, 1.0f / 720.0f);
    p = __builtin_fmaf(p, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    float e = __builtin_ldexpf(p, (int)n);
    // Keeps the series unconditional: without it the compiler turns the
    // select below back into a branch around the series.
    asm volatile("" : "+v"(e));
    return in_range ? e : (x != x ? x : 0.0f);
}

__device__ __forceinline__ float clamp127(float x) { return fminf(fmaxf(x, -127.0f), 127.0f); }

// Lane exchanges inside a row of 16 lanes through DPP (no LDS round trip).
// Applied in this order they pair lanes as a pairwise tree over the 16
// lanes: xor 1, xor 2 (quad_perm), then the two halves of each 8-lane group
// (row_half_mirror), then the two halves of the row (row_mirror).  After
// step L every lane holds the value of its aligned 2^L-lane block, combined
// exactly as the level-by-level pairwise sum does.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;
template <int CTRL>
__device__ __forceinline__ float dpp(float x)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float row16_max(float x)
{
    x = fmaxf(x, dpp<DPP_XOR1>(x));
    x = fmaxf(x, dpp<DPP_XOR2>(x));
    x = fmaxf(x, dpp<DPP_HALF_MIRROR>(x));
    return fmaxf(x, dpp<DPP_MIRROR>(x));
}
__device__ __forceinline__ float row16_tree_sum(float x)
{
    x = x + dpp<DPP_XOR1>(x);
    x = x + dpp<DPP_XOR2>(x);
    x = x + dpp<DPP_HALF_MIRROR>(x);
    return x + dpp<DPP_MIRROR>(x);
}
// Order-preserving integer key of a float (for non-NaN values: a < b as
// floats iff key(a) < key(b) as signed integers, with -0 below +0).  Maxima
// over keys need no NaN quieting and fuse with DPP lane moves.
__device__ __forceinline__ int fkey(float f)
{
    const int b = __float_as_int(f);
    return b ^ ((b >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float fkey_value(int k) { return __int_as_float(k ^ ((k >> 31) & 0x7fffffff)); }
template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) { return __builtin_amdgcn_mov_dpp(x, CTRL, 0xF, 0xF, true); }
__device__ __forceinline__ int row16_max_key(int x)
{
    x = max(x, dpp_i<DPP_XOR1>(x));
    x = max(x, dpp_i<DPP_XOR2>(x));
    x = max(x, dpp_i<DPP_HALF_MIRROR>(x));
    return max(x, dpp_i<DPP_MIRROR>(x));
}

// Maximum over the 64 lanes of a wave (the same value in every lane).
__device__ __forceinline__ float wave_max(float x)
{
    x = row16_max(x);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// A value that is the same in every lane (read from LDS after a barrier),
// moved to a scalar register so it does not occupy a VGPR.
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Tiles live in LDS as 128 key rows of 512 B, filled straight from HBM by
// LDS DMA (global_load_lds_dwordx4: one instruction moves 64 lanes x 16 B
// into 1 KiB of consecutive LDS).  Instruction r (0..7) of wave w moves the
// rows of keys 16w + r and 16w + 8 + r into row slots 16w + 2r and 16w + 2r
// + 1, so each lane follows one key through the wave's 8 instructions.
// Inside a slot the 16-byte chunks are XOR-swizzled with swz(slot), which
// keeps the DMA writes whole-row and makes both readers conflict-free: the
// QK operand reads (16 lanes = the 16 keys of a wave, one chunk each) and the
// transposed PV reads (16 lanes = 8 keys x two 8-byte halves of one chunk;
// neighbouring 16-lane groups use opposite halves of the banks).
__device__ __forceinline__ int slot_of(int key) { return (key & ~15) + 2 * (key & 7) + ((key >> 3) & 1); }
__device__ __forceinline__ int swz(int slot) { return ((slot >> 1) & 7) | (((slot ^ (slot >> 4)) & 1) << 3); }
__device__ __forceinline__ int tile_offset(int slot, int chunk) { return slot * D + ((chunk ^ swz(slot)) << 4); }

// MFMA row m of the 16-row operands: rows 4g..4g+3 hold heads 2g and 2g+1,
// each as {code, residual}.  Output lane group g then owns both rows of both
// of its heads.
__device__ __forceinline__ int row_of(int head, int residual) { return 4 * (head >> 1) + 2 * (head & 1) + residual; }

// Waits that do not imply a memory fence: LDS DMA of the next tile stays in
// flight across them.  vm_wait<N> returns once at most N of this wave's
// vector-memory operations are outstanding (they complete in issue order);
// lds_barrier makes this wave's LDS writes visible to the work-group.
template <int N_OUT>
__device__ __forceinline__ void vm_wait()
{
    static_assert(N_OUT == 0 || N_OUT == 8, "encoded waits");
    if (N_OUT == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
}
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// LDS DMA of 16 bytes per lane: lane l's 16 bytes at `src` land at LDS byte
// address lds + 16 l.  Written as inline assembly so that the compiler does
// not track it: its own tracking cannot tell the two ring buffers apart and
// would wait for the next tile's DMA before every LDS read.  The callers
// order these copies with vm_wait and lds_barrier instead.  M0 carries the
// LDS address (the compiler keeps nothing live in M0 in this file).  NT sets
// the non-temporal cache policy, for launches whose KV rows are read about
// once (decode: few query tokens per sequence).  Prefill launches, whose
// query tokens re-read the same rows from L2, keep the default policy.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <bool NT>
__device__ __forceinline__ void dma16(uint64_t src, uint32_t lds)
{
    if (NT)
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" :: "v"(src), "s"(lds) : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(src), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

// Query tokens per sequence slot up to which a launch's KV copies are
// non-temporal: C4 rows of two tokens' top-k lists rarely coincide; the C128
// tokens of one sequence all read the same compressed rows.
constexpr uint32_t STREAM_TOKENS_C4 = 4, STREAM_TOKENS_C128 = 1;
constexpr int QSTAGE = D + 16;   // row stride of the Q code staging area
constexpr int DMA_PER_TILE = N * D / 1024 / WAVES;   // LDS DMA instructions per wave and tile
static_assert(DMA_PER_TILE == 8, "vm_wait<8> covers one tile in flight");

// Small arrays first, so their LDS offsets fit instruction offset fields.
struct alignas(16) Shared {
    int32_t redmax[HEADS][WAVES];   // per-wave tile maxima (fkey)
    float redsum[HEADS][WAVES];     // per-wave weight sums
    float redsum1[HEADS][WAVES];    // joint rows: per-wave weight sums of the compressed tile
    float asc[2][HEADS];            // alpha * softmax_scale per kind
    int32_t scan[WAVES];
    int32_t misc[8];
    uint64_t listed[2];             // joint C4 rows: compressed rows 0-127 with multiplicity > 0
    int32_t mult[N];                // joint C4 rows: multiplicity of compressed row r among the top-k entries
    float bias[N];                  // joint C4 rows: log(multiplicity) of compressed list position j
    float scale[2][D];              // channel scales of the window / compressed cache
    int8_t p[16 * PROW];            // P codes [MFMA row][key]
    int32_t code[CODE_TILES * N];   // row codes of the resident tiles: page * 32 + row, -1 masked
    uint64_t addr[CODE_TILES * N];  // HBM address of each resident row (masked rows: an in-bounds dummy)
    int8_t tile[2][N * D];          // two K/V tiles (the DMA ring); Q code staging before the first tile
};
static_assert(2 * 16 * QSTAGE <= N * D, "Q staging fits in one tile buffer");
static_assert(offsetof(Shared, tile) % 16 == 0, "16-byte LDS DMA rows and tile reads");

struct Row {
    int32_t batch, position, first_ori, ori_count, count, list_len, t0, total;
};

// Partition states are exchanged between work-groups that may sit on
// different XCDs (each with its own L2).  They are written and read with
// buffer accesses carrying the sc1 cache policy (device-coherent: written
// through to, and read from, the point of coherence of all XCDs) instead of
// flushing and invalidating the whole L2 around a device-scope fence.
constexpr int SC1 = 16;                    // cache-policy operand: sc1
constexpr int SC0 = 1;                     // cache-policy operand: sc0 (miss the CU's L1, read the XCD's L2)
// Bits of the attention kernels' `fused` argument.  FUSED_MERGE: the last
// partition of a row folds it in the launch.  FUSED_XCD_LOCAL: work-groups
// whose blockIdx agree modulo 8 run on one XCD (checked once per device by
// the library's dispatch probe), so a row whose partitions all sit on one
// XCD exchanges its states through that XCD's L2 (sc0 stores and loads)
// instead of the device's point of coherence; its ticket stays
// device-coherent.
constexpr uint32_t FUSED_MERGE = 1, FUSED_XCD_LOCAL = 2;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_states(float *base)
{
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, 0x00020000);
}
// The raw buffer builtins move 32-bit integer words; floats travel as bits.
template <int POLICY>
__device__ __forceinline__ void state_store(float v, __amdgpu_buffer_rsrc_t r, int offset)
{
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, offset, 0, POLICY);
}
template <int POLICY>
__device__ __forceinline__ float state_load(__amdgpu_buffer_rsrc_t r, int offset)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, offset, 0, POLICY));
}
template <int POLICY>
__device__ __forceinline__ f32x4 state_load4(__amdgpu_buffer_rsrc_t r, int offset)
{
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, POLICY));
}

// Folds the S partition states of one query row (reference.py:317-323):
// top = max of the partition maxima; f_s = exp(max_s - top);
// out = bf16(sum_s num_s f_s / sum_s den_s f_s), lse = top + log(den).
// Thread = (head tid / 64, columns 8 (tid % 64) .. + 7) of a 512-thread
// group.  Partitions are folded in order.  MAXS bounds S at compile time so
// every load is issued before any is used (offsets of partitions past S are
// clamped to partition 0 and their values ignored); fold_row instantiates it
// exactly for 2-6 partitions (the five-or-three plan and short rows), since
// every clamped partition still costs its loads and its exponential, for 7-8
// at once, and above eight in groups (fold_states_wide).
template <int MAXS, int POLICY>
__device__ __forceinline__ void fold_states(const __amdgpu_buffer_rsrc_t states, int S, int tid,
                                            uint16_t *out_row, float *lse_row, int heads)
{
    const int h = tid >> 6, col = (tid & 63) * 8;
    const int head_base = h * PART_FLOATS * 4;
    const int part_step = HEADS * PART_FLOATS * 4;
    float ms[MAXS], ds[MAXS];
    f32x4 v0[MAXS], v1[MAXS];
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) {
        const int at = head_base + (sp < S ? sp : 0) * part_step;
        ms[sp] = state_load<POLICY>(states, at + 512 * 4);
        ds[sp] = state_load<POLICY>(states, at + 513 * 4);
        v0[sp] = state_load4<POLICY>(states, at + col * 4);
        v1[sp] = state_load4<POLICY>(states, at + (col + 4) * 4);
    }
    float top = ms[0];
#pragma unroll
    for (int sp = 1; sp < MAXS; ++sp) top = sp < S ? fmaxf(top, ms[sp]) : top;
    float f[MAXS], dsum = 0.0f;
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) {
        f[sp] = sk_expf_nonpos(ms[sp] - top);
        dsum = sp < S ? dsum + ds[sp] * f[sp] : dsum;
    }
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp)
        if (sp < S) {
            acc[0] = acc[0] + v0[sp].x * f[sp];
            acc[1] = acc[1] + v0[sp].y * f[sp];
            acc[2] = acc[2] + v0[sp].z * f[sp];
            acc[3] = acc[3] + v0[sp].w * f[sp];
            acc[4] = acc[4] + v1[sp].x * f[sp];
            acc[5] = acc[5] + v1[sp].y * f[sp];
            acc[6] = acc[6] + v1[sp].z * f[sp];
            acc[7] = acc[7] + v1[sp].w * f[sp];
        }
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = pack_bf16(acc[2 * e] / dsum, acc[2 * e + 1] / dsum);
    if (heads < HEADS && h >= heads) return;   // padding heads of the last group of eight
    *reinterpret_cast<v4i *>(out_row + h * D + col) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    if (lse_row && (tid & 63) == 0) lse_row[h] = top + logf(dsum);
}

// The same fold for more than eight partitions, in the same order: every
// partition maximum is loaded at once (MAX_SPLITS of them, clamped as
// above), then the partitions' sums and accumulators eight at a time, each
// group's loads issued before any is used.  Holding sixteen partitions'
// accumulators at once would spill registers in the attention kernel; a
// loop over the partitions one by one would wait on every load.
template <int POLICY>
__device__ __forceinline__ void fold_states_wide(const __amdgpu_buffer_rsrc_t states, int S, int tid,
                                                 uint16_t *out_row, float *lse_row, int heads)
{
    constexpr int CHUNK = 8;
    static_assert(MAX_SPLITS % CHUNK == 0, "whole groups of partitions");
    const int h = tid >> 6, col = (tid & 63) * 8;
    const int head_base = h * PART_FLOATS * 4;
    const int part_step = HEADS * PART_FLOATS * 4;
    float ms[MAX_SPLITS];
#pragma unroll
    for (int sp = 0; sp < (int)MAX_SPLITS; ++sp)
        ms[sp] = state_load<POLICY>(states, head_base + (sp < S ? sp : 0) * part_step + 512 * 4);
    float top = ms[0];
#pragma unroll
    for (int sp = 1; sp < (int)MAX_SPLITS; ++sp) top = sp < S ? fmaxf(top, ms[sp]) : top;
    float dsum = 0.0f;
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < (int)MAX_SPLITS; c += CHUNK) {
        if (c >= S) break;
        float ds[CHUNK];
        f32x4 v0[CHUNK], v1[CHUNK];
#pragma unroll
        for (int k = 0; k < CHUNK; ++k) {
            const int at = head_base + (c + k < S ? c + k : 0) * part_step;
            ds[k] = state_load<POLICY>(states, at + 513 * 4);
            v0[k] = state_load4<POLICY>(states, at + col * 4);
            v1[k] = state_load4<POLICY>(states, at + (col + 4) * 4);
        }
#pragma unroll
        for (int k = 0; k < CHUNK; ++k)
            if (c + k < S) {
                const float f = sk_expf_nonpos(ms[c + k] - top);
                dsum = dsum + ds[k] * f;
                acc[0] = acc[0] + v0[k].x * f;
                acc[1] = acc[1] + v0[k].y * f;
                acc[2] = acc[2] + v0[k].z * f;
                acc[3] = acc[3] + v0[k].w * f;
                acc[4] = acc[4] + v1[k].x * f;
                acc[5] = acc[5] + v1[k].y * f;
                acc[6] = acc[6] + v1[k].z * f;
                acc[7] = acc[7] + v1[k].w * f;
            }
    }
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = pack_bf16(acc[2 * e] / dsum, acc[2 * e + 1] / dsum);
    if (heads < HEADS && h >= heads) return;
    *reinterpret_cast<v4i *>(out_row + h * D + col) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    if (lse_row && (tid & 63) == 0) lse_row[h] = top + logf(dsum);
}

template <int POLICY>
__device__ __forceinline__ void fold_row(const __amdgpu_buffer_rsrc_t states, int S, int tid, uint16_t *out_row,
                                         float *lse_row, int heads = HEADS)
{
    if (S <= 2) fold_states<2, POLICY>(states, S, tid, out_row, lse_row, heads);
    else if (S == 3) fold_states<3, POLICY>(states, S, tid, out_row, lse_row, heads);
    else if (S == 4) fold_states<4, POLICY>(states, S, tid, out_row, lse_row, heads);
    else if (S == 5) fold_states<5, POLICY>(states, S, tid, out_row, lse_row, heads);
    else if (S == 6) fold_states<6, POLICY>(states, S, tid, out_row, lse_row, heads);
    else if (S <= 8) fold_states<8, POLICY>(states, S, tid, out_row, lse_row, heads);
    else fold_states_wide<POLICY>(states, S, tid, out_row, lse_row, heads);
}

// SLOTS: the original kind is the explicit physical slot list of the row
// (oriIndices [tokens][1][oriTopk], reference.py:236-239 and 285), every
// entry in its list place, entries outside [0, oriPages * 32) masked, in
// ceil(oriTopk / 128) tiles; otherwise it is the SWA window through the
// block table.
// ANYH: p.heads is any of 1..128.  A work-group takes one group of eight
// heads of a query row (rows of the launch = tokens x ceil(heads / 8));
// heads past p.heads in the last group are computed on zero Q and never
// written.  Above eight heads the Q and P residual codes are zero
// (reference.py:221-222: residual quantization only for <= 8 heads), which
// leaves every other operation as it is.  Without ANYH, heads == 8.
template <int RATIO, bool DEBUG, bool SLOTS, bool ANYH, bool STREAM, bool JOINT>
__global__ void __launch_bounds__(THREADS, 1)   // one work-group per CU: the 128 KiB tile ring fills the LDS
c8_attention(const uint64_t cu_q, const uint64_t seq_lens, const uint64_t q_base, const uint64_t cmp_indices,
             const uint32_t batch_arg, const uint32_t topk_arg, const uint32_t heads_arg, const uint32_t splits,
             const uint32_t rows_arg, const uint32_t grid, const SharedKVArgs p, const SharedKVDebug dbg,
             const uint32_t fused)
{
    __shared__ Shared s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, n = lane & 15;

    // XCD-aware order: consecutive work items (the partitions of one row,
    // then the next row) stay on one XCD and share its L2: XCD x takes the
    // items [x G / 8, (x + 1) G / 8).
    const uint32_t G = grid;
    const uint32_t item = (blockIdx.x & 7u) * (G >> 3) + (blockIdx.x >> 3);
    const uint32_t items = rows_arg * splits;
    if (item >= items) return;
    const int H = ANYH ? (int)heads_arg : HEADS;                 // heads of a query token
    const int HG = ANYH ? (H + HEADS - 1) / HEADS : 1;           // groups of eight
    const bool resid = !ANYH || H <= HEADS;
    // The launch's plan: `splits` partitions per row over rows_arg rows.
    // rows.  The work item's row under that plan is loaded at once; with
    // graph padding the device re-plans (below) and may move it.
    int32_t S = (int32_t)splits;
    int32_t qrow = (int32_t)(item / splits);                     // (token, head group)
    int32_t t = ANYH ? qrow / HG : qrow;
    int32_t hbase = ANYH ? HEADS * (qrow % HG) : 0;
    int hlive = ANYH ? (H - hbase < HEADS ? H - hbase : HEADS) : HEADS;
    int32_t part = (int32_t)(item % splits);
    // Whether every partition of this work item's row runs on this
    // work-group's XCD: items [x G / 8, (x + 1) G / 8) are on XCD x.
    const uint32_t per_xcd_items = G >> 3;
    auto same_xcd = [&](uint32_t row, uint32_t parts) {
        return (row * parts) / per_xcd_items == (row * parts + parts - 1) / per_xcd_items;
    };
    bool together = same_xcd((uint32_t)qrow, splits);

    // ---- prologue: the loads the selection needs, issued together ----
    // cu_q, seq_lens, q_base, cmp_indices, batch_arg, topk_arg, heads_arg,
    // splits, rows_arg and grid are the leading kernel arguments (copies of
    // argument-block fields) that arrive preloaded in SGPRs.
    const __attribute__((address_space(1))) int32_t *cu = gptr<int32_t>(cu_q);
    const __attribute__((address_space(1))) int32_t *lens = gptr<int32_t>(seq_lens);
    const int batch_n = (int)batch_arg;
    // Request b's (cu[b], cu[b+1], len[b]) for b = tid (more in the loops below).
    // Unconditional (threads past the batch read request 0 and ignore it),
    // so the wait for these three loads leaves the later ones in flight.
    const int mine_b = tid < batch_n ? tid : 0;
    const int my_cu0 = cu[mine_b], my_cu1 = cu[mine_b + 1], my_len = lens[mine_b];
    // Q row t: 8 heads x 512 BF16; thread = head (= wave), channels lane * 8.
    const int qd0 = lane * 8;
    v4i qv = {0, 0, 0, 0};
    if (!ANYH || wave < hlive) qv = *gptr<v4i>(q_base + (((uint64_t)t * H + hbase + wave) * D + qd0) * 2);
    // C4 index entries 2 tid, 2 tid + 1 of row t.
    int ix[2] = {-1, -1};
    if (RATIO == 4) {
        const int topk = (int)topk_arg;
        const __attribute__((address_space(1))) int32_t *row_ix = gptr<int32_t>(cmp_indices) + (int64_t)t * topk;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            if (tid * 2 + i < topk) ix[i] = row_ix[tid * 2 + i];
    }

    // ---- live shape (attention_impl.h:121-137) ----
    // The last request with seq_len > 0 and cu_q >= 0 ends the live batch;
    // its cu_q end bounds the live tokens.  The longest of those requests
    // bounds the rows' tile counts; kernels that choose joint rows from it
    // take it in the same pass.
    if (tid == 0) { s.misc[0] = 0; s.misc[1] = -1; s.misc[2] = 0; s.misc[6] = 0; }
    __syncthreads();
    for (int b = tid; b < batch_n; b += THREADS) {
        const int len = b == tid ? my_len : lens[b];
        const int c1 = b == tid ? my_cu1 : cu[b + 1];
        if (len > 0 && c1 >= 0) {
            atomicMax(&s.misc[0], b + 1);
            if (JOINT) atomicMax(&s.misc[6], len);
        }
    }
    __syncthreads();
    const int live_batch = uni(s.misc[0]);
    // The live end and the request holding token t of the launch plan's row.
    auto find_request = [&](int token, bool first) {
        for (int b = tid; b < live_batch; b += THREADS) {
            const int c0 = b == tid ? my_cu0 : cu[b];
            const int c1 = b == tid ? my_cu1 : cu[b + 1];
            const int len = b == tid ? my_len : lens[b];
            if (c0 <= token && token < c1) {
                s.misc[1] = b;
                s.misc[3] = len;
                s.misc[4] = c1;
            }
            if (first && b == live_batch - 1) s.misc[2] = c1;
        }
        __syncthreads();
    };
    find_request(t, true);
    const int end = live_batch ? uni(s.misc[2]) : 0;
    const int live_tokens = end <= 0 ? 0 : (end < (int)p.tokens ? end : (int)p.tokens);

    // ---- device plan (c4_wide.h:16-41 of the reference chooses from the
    // live shape too) ----  When graph padding leaves live rows below the
    // launch's capacity, the idle work items become more partitions of the
    // live rows: the host's rule for an eager launch of that many rows (5
    // partitions while rows x 5 fit the CUs, else 3, at most CUs / rows and
    // the longest live row's tile count), capped by items / live rows and
    // never below the launch's own plan.  Each work item also zero-fills one
    // padding row.  The rule is c8_attention.device_splits on the host; the
    // separate merge launch (not fused) keeps the launch plan.
    const int32_t rows_cap = (int32_t)rows_arg;
    const int32_t live_rows = live_tokens * HG;
    // The longest live sequence bounds the rows' tile counts (one scan, only
    // where a plan needs it).
    int longest = JOINT ? uni(s.misc[6]) : -1;
    auto longest_live = [&]() {
        if (longest < 0) {
            for (int b = tid; b < live_batch; b += THREADS) {
                const int len = b == tid ? my_len : lens[b];
                if (len > 0 && (b == tid ? my_cu1 : cu[b + 1]) >= 0) atomicMax(&s.misc[6], len);
            }
            __syncthreads();
            longest = uni(s.misc[6]);
        }
        return longest;
    };
    // Joint plan (JOINT: every C128 kernel, and C4 kernels launched for
    // block tables of at most one tile of compressed rows per sequence):
    // when every live row's window and compressed lists fit one tile each
    // (at most N compressed rows: longest sequence / RATIO <= N),
    // the launch runs as one partition per row and those rows take one
    // softmax over both kinds, as the reference device's one-split C128
    // plans (c128.cpp:79-105, attention_impl.h:94-100) and its short C4 task
    // batches (c4.cpp:35-58, task_batch.h) do.  Work items of the other
    // partitions have nothing to do.  A launch with a separate merge keeps
    // its plan; c8_attention.device_splits mirrors the rule.
    bool joint_launch = false;
    if (JOINT && !DEBUG && !SLOTS && resid && (fused || S == 1) && live_rows > 0 &&
        longest_live() / RATIO <= N) {
        if (part != 0) return;
        S = 1;
        joint_launch = true;
    } else if (fused && live_rows < rows_cap) {
        const int32_t pad = live_rows + (int32_t)item;
        if (pad < rows_cap) {   // zero-fill padding row `pad` (attention_impl.h:443-460)
            const int32_t pt = ANYH ? pad / HG : pad, ph = ANYH ? HEADS * (pad % HG) : 0;
            const int pl = ANYH ? (H - ph < HEADS ? H - ph : HEADS) : HEADS;
            uint16_t *o = reinterpret_cast<uint16_t *>(p.out) + ((int64_t)pt * H + ph) * D;
            if (!ANYH || tid < pl * (D / 8)) reinterpret_cast<v4i *>(o)[tid] = v4i{0, 0, 0, 0};
            if (p.lse && tid < pl) reinterpret_cast<float *>(p.lse)[(int64_t)pt * H + ph + tid] = 0.0f;
        }
        if (live_rows == 0) return;
        longest_live();
        int tiles = SLOTS ? ((int)p.oriTopk + N - 1) / N : 1;
        if (RATIO == 4) {
            const int cnt = longest / 4 < (int)topk_arg ? longest / 4 : (int)topk_arg;
            tiles += (cnt + N - 1) / N;
        } else if (RATIO == 128) {
            tiles += (longest / 128 + N - 1) / N;
        }
        int32_t plan = live_rows * PLAN_FEW <= PLAN_CUS ? PLAN_FEW : PLAN_MANY;
        const int32_t fit = PLAN_CUS / live_rows > 1 ? PLAN_CUS / live_rows : 1;
        const int32_t room = (int32_t)(items / (uint32_t)live_rows);
        if (live_rows * tiles <= PLAN_ONE_TILE && tiles <= (int32_t)MAX_SPLITS && tiles <= room) plan = tiles;
        plan = plan < fit ? plan : fit;
        plan = plan < tiles ? plan : tiles;
        plan = plan < room ? plan : room;
        plan = plan > S ? plan : S;
        // Placement of the live work items: every XCD takes a contiguous
        // eighth of the live rows (rows [x R / 8, (x + 1) R / 8) on XCD x,
        // each with all its partitions), so that a padded launch spreads
        // over the whole chip like an eager launch of its live rows, when
        // every XCD has the work-groups for its share (the fullest XCD holds
        // ceil(R / 8) rows; XCD 7 loses the grid's rounding work-groups);
        // otherwise item i takes row i / plan on the launch's own order.
        // (XCD x holds min(G / 8, items - x G / 8) work-groups; usable is
        // the fewest, that of XCD 7, or negative when XCD 7 holds none.)
        int32_t row;
        const int32_t per_xcd = (int32_t)(G >> 3), usable = per_xcd - (int32_t)(G - items);
        if ((live_rows + 7) / 8 * plan <= usable) {
            const int32_t x = (int32_t)(blockIdx.x & 7u), j = (int32_t)(blockIdx.x >> 3);
            row = x * live_rows / 8 + j / plan;
            if (row >= (x + 1) * live_rows / 8) return;
            part = j % plan;
            together = true;
        } else {
            if (item >= (uint32_t)(live_rows * plan)) return;
            row = (int32_t)(item / (uint32_t)plan);
            part = (int32_t)(item % (uint32_t)plan);
            together = same_xcd((uint32_t)row, (uint32_t)plan);
        }
        S = plan;
        if (row != qrow) {
            // The work item moved to another row: load that row's Q and indices.
            qrow = row;
            t = ANYH ? qrow / HG : qrow;
            hbase = ANYH ? HEADS * (qrow % HG) : 0;
            hlive = ANYH ? (H - hbase < HEADS ? H - hbase : HEADS) : HEADS;
            qv = v4i{0, 0, 0, 0};
            if (!ANYH || wave < hlive) qv = *gptr<v4i>(q_base + (((uint64_t)t * H + hbase + wave) * D + qd0) * 2);
            if (RATIO == 4) {
                const int topk = (int)topk_arg;
                const __attribute__((address_space(1))) int32_t *row_ix = gptr<int32_t>(cmp_indices) + (int64_t)t * topk;
#pragma unroll
                for (int i = 0; i < 2; ++i) ix[i] = tid * 2 + i < topk ? row_ix[tid * 2 + i] : -1;
            }
            if (tid == 0) s.misc[1] = -1;
            __syncthreads();
            find_request(t, false);
        }
    }
    // The work item (query row qrow, partition part) from its row request
    // onwards.  joint_c4 (a compile-time flag): the launch is a joint-plan C4
    // launch, whose rows take the joint route; C4 kernels with joint rows
    // compiled in hold one specialized copy for such launches and one for
    // tiled launches, so the tiled copy is the same code as in kernels
    // without them.
    auto run_row = [&](auto joint_c4) {
        constexpr bool JC4 = decltype(joint_c4)::value;
        // Every metadata load has landed: said explicitly (vmcnt(0)) so that the
        // compiler's own wait tracking does not hold back the block-table reads
        // issued next for these registers.
        __builtin_amdgcn_s_waitcnt(0x0F70);
        const int batch = uni(s.misc[1]);
        uint16_t *out_row = reinterpret_cast<uint16_t *>(p.out) + ((int64_t)t * H + hbase) * D;
        float *lse_row = p.lse ? reinterpret_cast<float *>(p.lse) + (int64_t)t * H + hbase : nullptr;
        // A row without keys is zero-filled by partition 0: output and LSE, and
        // with a separate merge launch its partition count (0: nothing to fold).
        auto zero_row = [&]() {
            if (part != 0) return;
            if (!ANYH || tid < hlive * (D / 8)) reinterpret_cast<v4i *>(out_row)[tid] = v4i{0, 0, 0, 0};
            if (lse_row && tid < hlive) lse_row[tid] = 0.0f;
            if (S > 1 && !fused && tid == 0)
                reinterpret_cast<float *>(p.partial)[(int64_t)qrow * S * HEADS * PART_FLOATS + FOLD_SLOT] = 0.0f;
        };
        if (t >= live_tokens || batch < 0) {
            zero_row();   // graph padding rows (attention_impl.h:443-460)
            return;
        }
        // Sinks and the scales of both kinds (kind = tid / 256, 2 channels per
        // thread): their addresses come from the argument block, which is read
        // while the metadata above is in flight, so they are requested only now;
        // the scales go to LDS after the block-table reads have been issued.
        const __attribute__((address_space(1))) float *sinks = gptr<float>(p.sinks);
        const float sink0 = (!ANYH || 2 * g < hlive) ? sinks[hbase + 2 * g] : 0.0f;
        const float sink1 = (!ANYH || 2 * g + 1 < hlive) ? sinks[hbase + 2 * g + 1] : 0.0f;
        const f32x2 scale_pair = *gptr<f32x2>(((tid >> 8) && RATIO != 1 ? p.cmpScale : p.oriScale) +
                                              (uint64_t)((tid & 255) * 2) * 4);

        // ---- selection (attention_impl.h:58-73, reference.py:228-253) ----
        Row m;
        m.batch = batch;
        m.position = uni(s.misc[3]) - uni(s.misc[4]) + t;
        m.first_ori = m.position + 1 > WINDOW ? m.position + 1 - WINDOW : 0;
        m.ori_count = m.position + 1 - m.first_ori;
        if (m.ori_count < 0) m.ori_count = 0;
        if (SLOTS) {
            m.first_ori = 0;
            m.ori_count = (int)p.oriTopk;
        }
        m.count = RATIO == 1 ? 0 : (m.position + 1) / RATIO;
        // Global-space views: flat loads would also hold the LDS counter that the
        // fence-free barriers below wait on.
        const __attribute__((address_space(1))) int32_t *otab = gptr<int32_t>(p.oriTable) + (int64_t)m.batch * p.oriTableWidth;
        const __attribute__((address_space(1))) int32_t *ctab = gptr<int32_t>(p.cmpTable) + (int64_t)m.batch * p.cmpTableWidth;
        // C4: every block-table read of the row (the window tile, held by
        // partition 0, and the thread's two index entries) is issued here, so
        // the compaction scan below runs while they are in flight.  A C4 row
        // has at most 1 + MAX_LIST / N <= CODE_TILES tiles: one chunk of codes
        // (explicit slots read theirs per chunk, below).
        const __attribute__((address_space(1))) int32_t *oslots =
            gptr<int32_t>(p.oriIndices) + (int64_t)t * p.oriTopk;
        int wpage = -1, widx = -1, cpage_raw[2] = {-1, -1};
        if (RATIO == 4) {
            if (!SLOTS && part == 0 && tid < m.ori_count) {
                const int idx = m.first_ori + tid;
                if (idx / BLOCK_ROWS < (int)p.oriTableWidth) {
                    widx = idx;
                    wpage = otab[idx / BLOCK_ROWS];
                }
            }
#pragma unroll
            for (int e = 0; e < 2; ++e)
                if (ix[e] >= 0 && ix[e] < m.count && ix[e] / BLOCK_ROWS < (int)p.cmpTableWidth)
                    cpage_raw[e] = ctab[ix[e] / BLOCK_ROWS];
        }
        static_assert(1 + MAX_LIST / N <= CODE_TILES, "a C4 row's codes fit one chunk");
        int ipos[2] = {-1, -1};   // list position of each owned C4 entry (-1: none)
        if (RATIO == 4) {
            const int topk = (int)p.topk;
            const bool compact = m.count < topk && topk <= MAX_LIST;   // reference.py:250
            bool ok[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) ok[i] = ix[i] >= 0 && ix[i] < m.count;
            if (compact) {
                // Entry 2 tid + i goes to place (valid entries of lower lanes and
                // waves) + (entry 0 of this lane, for i = 1): two ballots, counted
                // below the lane with mbcnt.
                const uint64_t v0 = __ballot(ok[0]), v1 = __ballot(ok[1]);
                const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(v0 >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)v0, 0u)) +
                                  (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(v1 >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)v1, 0u));
                if (lane == 0) s.scan[wave] = __popcll(v0) + __popcll(v1);
                lds_barrier();                    // no fence: the table reads stay in flight
                int at = below, total = 0;
#pragma unroll
                for (int w = 0; w < WAVES; ++w) {
                    at += w < wave ? s.scan[w] : 0;
                    total += s.scan[w];
                }
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    if (ok[i]) ipos[i] = at++;
                m.list_len = uni(total);
            } else {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int j = tid * 2 + i;
                    if (j < topk) ipos[i] = j;
                    if (!ok[i]) ix[i] = -1;        // hole: a masked column in place
                }
                m.list_len = topk;
            }
        } else if (RATIO == 128) {
            m.list_len = m.count > 0 ? m.count : 0;
        } else {
            m.list_len = 0;   // window only
        }
        m.t0 = (m.ori_count + N - 1) / N;
        m.total = m.t0 + (m.list_len + N - 1) / N;
        // Joint sparse row (C4, reference.py:246-267 with joint_sparse; JOINT
        // instantiations only): in a launch of the joint plan (every live row's
        // compressed rows fit one tile: count <= N) a row's compressed list is
        // dense: every row below
        // count that some valid top-k entry names, once, in row order, with
        // log(multiplicity) added to its logits (built with the row codes,
        // below).  reference.py switches every C4 row of such a plan to the
        // dense list, so a launch with a longer row has no joint C4 rows (the
        // reference device decides per launch too, c4.cpp:35-58).  A joint C4
        // row is two tiles even when it lists no compressed row (reference.py:257
        // takes the joint route then too): its compressed tile is then all
        // masked.  The joint route rounds the PV dequantization differently from
        // the tiled one, so the row keeps it.
        const bool joint4 = RATIO == 4 && JC4 && m.count <= N;
        if (joint4 && m.position >= 0) m.total = 2;
        const int my_tiles = m.total > part ? (m.total - part + S - 1) / S : 0;   // tiles part, part + S, ...
        // A live row's window list holds at least its own position, so it has a
        // tile, unless its request lists more query tokens than its sequence
        // length (a negative position, which reference.py:104-105 rejects): that
        // row is zero-filled, explicit original slots or not.
        if (m.total == 0 || m.position < 0) {
            zero_row();
            return;
        }
        // Partitions that own no tile (part >= total) hold the initial state
        // (max = sink <= every owning partition's max, numerator and denominator
        // 0), which folds to exactly nothing: they publish nothing, and a row
        // whose tiles all sit in partition 0 is finalized by it directly.  The
        // numbers equal the fold over all S partitions bit for bit.
        const int folded = S < m.total ? S : m.total;    // partitions that own tiles (>= 1)
        if (part >= folded) return;
        // Joint row (reference.py:254-267 with joint_dense for C128, joint_sparse
        // for C4; the reference device's two-kind pipeline, attention_impl.h:
        // 94-100, and C4 task batches): a row run as one partition whose window
        // and compressed lists each fit one tile takes one softmax over both
        // kinds (joint_quantized_row, reference.py:175-207) instead of two
        // online tiles.  Tile 0 holds the window's keys in order, tile 1 the
        // compressed list's, the order in which the reference concatenates
        // them; the weight sum is one pairwise tree per kind, added in kind
        // order.  Explicit original slots, more than eight heads (no residual
        // codes) and the debug entry keep the tiled plan.
        const bool joint = RATIO == 128 ? !DEBUG && !SLOTS && resid && S == 1 && m.t0 == 1 && m.list_len >= 1 &&
                                              m.list_len <= N
                                        : joint4 && m.total == 2;

        // ---- per-lane softmax state for heads 2g and 2g+1 ----
        float mx[2] = {sink0, sink1}, den[2], num[2][4];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            den[hh] = part == 0 ? 1.0f : 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) num[hh][j] = 0.0f;
        }

        // PV integers of the last computed tile, awaiting the FP32 epilogue
        // (reference.py:313-316): num = num * factor + (V_hi + V_lo/127) * scale/127.
        v4i held_acc[4];
        float held_sc[4], held_factor[2];
        bool held = false;
        auto epilogue = [&]() {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float dots = (float)held_acc[j][2 * hh];
                    dots = dots + (float)held_acc[j][2 * hh + 1] * (float)(1.0 / 127.0);
                    const float pv = dots * held_sc[j] * (float)(1.0 / 127.0);
                    num[hh][j] = num[hh][j] * held_factor[hh] + pv;
                }
            }
            held = false;
        };

        const int positions = 128 + (int)dbg.cmpCapacity;
        const int c0 = 64 * wave;       // this wave's 64 PV output columns: c0 + 16 j + n

        // Q folding and residual split for both kinds (reference.py:274-279),
        // done once while the first tile's rows are in flight.  Thread = head
        // `wave`, channels qd0 .. qd0 + 7.  Codes are staged in tile buffer 1
        // (before any tile is requested into it) and picked up in the MFMA A
        // layout.
        v4i qa0[8], qa1[8];   // Q codes per 64-byte D block, window / compressed kind
        // Its inputs pass through opaque copies, so the compiler computes the
        // encode where it is called instead of ahead of the row codes.
        auto encode_q = [&](bool want0, bool want1) {
            v4i qx = qv;
            int lx = lane;
            asm volatile("" : "+v"(qx), "+v"(lx));
            const int qe0 = lx * 8, ne = lx & 15, ge = lx >> 4;
            const uint32_t qw[4] = {(uint32_t)qx.x, (uint32_t)qx.y, (uint32_t)qx.z, (uint32_t)qx.w};
#pragma unroll
            for (int kind = 0; kind < 2; ++kind) {
                if (!(kind ? want1 : want0)) continue;
                const float *scale = s.scale[kind] + qe0;
                float f[8];
                float amax = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    f[e] = bf16_to_f32((qw[e >> 1] >> (16 * (e & 1))) & 0xffffu) * scale[e];
                    amax = fmaxf(amax, fabsf(f[e]));
                }
                amax = wave_max(amax);              // the head's 512 channels
                float alpha = amax * (float)(1.0 / 127.0);
                alpha = alpha < 1e-12f ? 1e-12f : alpha;
                const float inv = 1.0f / alpha;
                uint32_t hiw[2] = {0, 0}, low[2] = {0, 0};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float x = clamp127(f[e] * inv);
                    const float hi = __builtin_rintf(x);
                    const float lo = resid ? __builtin_rintf((x - hi) * 127.0f) : 0.0f;
                    hiw[e >> 2] |= ((uint32_t)(int32_t)hi & 0xffu) << (8 * (e & 3));
                    low[e >> 2] |= ((uint32_t)(int32_t)lo & 0xffu) << (8 * (e & 3));
                }
                int8_t *stage = s.tile[1] + kind * 16 * QSTAGE;
                *reinterpret_cast<u32x2 *>(stage + row_of(wave, 0) * QSTAGE + qe0) = u32x2{hiw[0], hiw[1]};
                *reinterpret_cast<u32x2 *>(stage + row_of(wave, 1) * QSTAGE + qe0) = u32x2{low[0], low[1]};
                if (lane == 0) s.asc[kind][wave] = alpha * p.softmaxScale;
                if (DEBUG) {
                    if (dbg.qcodes) {
                        int8_t *qc = reinterpret_cast<int8_t *>(dbg.qcodes) + (((int64_t)t * 2 + kind) * 16) * D;
                        *reinterpret_cast<u32x2 *>(qc + wave * D + qe0) = u32x2{hiw[0], hiw[1]};
                        *reinterpret_cast<u32x2 *>(qc + (8 + wave) * D + qe0) = u32x2{low[0], low[1]};
                    }
                    if (dbg.alpha && lane == 0)
                        reinterpret_cast<float *>(dbg.alpha)[((int64_t)t * 2 + kind) * 8 + wave] = alpha;
                }
            }
            lds_barrier();
            const int8_t *st0 = s.tile[1], *st1 = s.tile[1] + 16 * QSTAGE;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                qa0[jj] = want0 ? *reinterpret_cast<const v4i *>(st0 + ne * QSTAGE + 64 * jj + 16 * ge) : v4i{0, 0, 0, 0};
                qa1[jj] = want1 ? *reinterpret_cast<const v4i *>(st1 + ne * QSTAGE + 64 * jj + 16 * ge) : v4i{0, 0, 0, 0};
            }
        };

        // LDS DMA of resident tile `i` into ring buffer `buf`: 8 instructions per
        // wave, always all 64 lanes (masked keys read a harmless in-bounds
        // address instead), so each tile is exactly DMA_PER_TILE vector-memory
        // operations per wave for vm_wait.
        // Instructions [r0, r0 + count) of the tile's DMA.  The row addresses
        // of a batch are read before its first copy is issued (each copy is a
        // compiler barrier for LDS accesses).
        auto issue_rows = [&](int i, int buf, int r0, int count) {
            const int h = lane >> 5, c = lane & 31;
            typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
            const u64x2 *rows = reinterpret_cast<const u64x2 *>(s.addr + i * N + 16 * wave + 8 * h + r0);   // keys 16 wave + 8 h + r
            u64x2 ra[DMA_PER_TILE / 2];
#pragma unroll
            for (int r = 0; r < DMA_PER_TILE / 2; ++r)
                if (2 * r < count) ra[r] = rows[r];
            const uint32_t dst = (uint32_t)(uintptr_t)(lds_i8 *)(s.tile[buf]) + 16 * wave * D;
            const int hx = (h ^ wave) & 1;
#pragma unroll
            for (int k = 0; k < DMA_PER_TILE; ++k) {
                if (k >= count) break;
                const int r = r0 + k;
                const int chunk = c ^ r ^ (hx << 3);   // swz(16 wave + 2 r + h)
                dma16<STREAM>(ra[k >> 1][k & 1] + (uint32_t)(chunk << 4), (uint32_t)uni((int)(dst + 2 * r * D)));
            }
        };
        auto issue_tile = [&](int i, int buf) { issue_rows(i, buf, 0, DMA_PER_TILE); };
        // The next tile's copies are spread over four points of the current
        // tile's body, two instructions each, so no wave stalls behind a full
        // tile's worth of queued copies.
        constexpr int DMA_STEP = DMA_PER_TILE / 4;

        // A C4 row without explicit slots has one chunk of codes: saying so lets
        // the compiler end the live ranges of its selection values there.
        constexpr bool ONE_CHUNK = RATIO == 4 && !SLOTS;
        for (int first = 0; first < my_tiles && (!ONE_CHUNK || first == 0); first += CODE_TILES) {
            const int ntiles = my_tiles - first < CODE_TILES ? my_tiles - first : CODE_TILES;
            // ---- row codes of partition tiles [first, first + ntiles) ----
            for (int i = tid; i < ntiles * N; i += THREADS) {
                s.code[i] = -1;
                s.addr[i] = p.q;              // masked rows: DMA reads 512 B of Q, never used
            }
            // Window / C128 rows: at most CODE_TILES * N / THREADS entries per
            // thread, all block-table reads issued before any is used.  Rows
            // whose logical page lies outside the block table, or whose physical
            // page is negative or (window cache) past the pool, stay masked.
            constexpr int PER = CODE_TILES * N / THREADS;
            int tpage[PER], tidx[PER];
#pragma unroll
            for (int e = 0; e < PER; ++e) {
                const int i = tid + e * THREADS;
                tidx[e] = -1;
                tpage[e] = -1;
                if (RATIO == 4 && !SLOTS) {       // read before the compaction scan
                    if (e == 0) {
                        tidx[0] = widx;
                        tpage[0] = wpage;
                    }
                    continue;
                }
                if (i >= ntiles * N) continue;
                const int k = part + S * (first + i / N), r = i % N;
                if (SLOTS && k < m.t0) {
                    const int j = k * N + r;      // place in the slot list
                    if (j < m.ori_count) {
                        tidx[e] = j;
                        tpage[e] = oslots[j];     // the physical slot
                    }
                } else if (k < m.t0) {
                    if (r < m.ori_count) {
                        const int idx = m.first_ori + r;
                        if (idx / BLOCK_ROWS < (int)p.oriTableWidth) {
                            tidx[e] = idx;
                            tpage[e] = otab[idx / BLOCK_ROWS];
                        }
                    }
                } else if (RATIO == 128) {
                    const int idx = (k - m.t0) * N + r;
                    if (idx < m.list_len && idx / BLOCK_ROWS < (int)p.cmpTableWidth) {
                        tidx[e] = idx;
                        tpage[e] = ctab[idx / BLOCK_ROWS];
                    }
                }
            }
            int cslot[2] = {-1, -1};
            if (RATIO == 4 && !joint) {       // joint rows take the dense list (below)
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    if (ipos[e] < 0 || ix[e] < 0) continue;
                    const int k = m.t0 + ipos[e] / N;
                    if (k < part || (k - part) % S) continue;
                    const int i = (k - part) / S - first;
                    if (i < 0 || i >= ntiles || ix[e] / BLOCK_ROWS >= (int)p.cmpTableWidth) continue;
                    cslot[e] = i * N + ipos[e] % N;
                }
            }
            if (first == 0) *reinterpret_cast<f32x2 *>(&s.scale[tid >> 8][(tid & 255) * 2]) = scale_pair;
            if (RATIO == 4 && joint && tid < N) s.mult[tid] = 0;
            lds_barrier();                    // the -1 fill is complete before the writes below
#pragma unroll
            for (int e = 0; e < PER; ++e) {
                if (tidx[e] < 0) continue;
                const int i = tid + e * THREADS;
                const bool window = part + S * (first + i / N) < m.t0;
                if (SLOTS && window) {
                    const int slot = tpage[e];
                    if (slot >= 0 && (uint32_t)slot < p.oriPages * BLOCK_ROWS) {
                        s.code[i] = slot;
                        s.addr[i] = p.ori + (uint64_t)(slot / BLOCK_ROWS) * p.oriStride + (uint64_t)((slot % BLOCK_ROWS) * D);
                    }
                    continue;
                }
                const bool ok = tpage[e] >= 0 && (!window || (uint32_t)tpage[e] < p.oriPages);
                if (ok) {
                    s.code[i] = tpage[e] * BLOCK_ROWS + tidx[e] % BLOCK_ROWS;
                    s.addr[i] = (window ? p.ori : p.cmp) + (uint64_t)tpage[e] * (window ? p.oriStride : p.cmpStride) +
                                (uint64_t)((tidx[e] % BLOCK_ROWS) * D);
                }
            }
            if (RATIO == 4) {
#pragma unroll
                for (int e = 0; e < 2; ++e)
                    if (cslot[e] >= 0 && cpage_raw[e] >= 0) {
                        s.code[cslot[e]] = cpage_raw[e] * BLOCK_ROWS + ix[e] % BLOCK_ROWS;
                        s.addr[cslot[e]] = p.cmp + (uint64_t)cpage_raw[e] * p.cmpStride + (uint64_t)((ix[e] % BLOCK_ROWS) * D);
                    }
                if (joint) {
                    // Tile 1 = the dense compressed list (reference.py:246-249):
                    // each row's multiplicity among the valid entries, then the
                    // listed rows (multiplicity > 0) in row order.  The owner of
                    // an entry writes its row's code at the row's list place
                    // (entries naming one row write the same code), from the
                    // table entry it read for the tiled plan; thread r writes
                    // row r's bias.
#pragma unroll
                    for (int e = 0; e < 2; ++e)
                        if (ix[e] >= 0 && ix[e] < m.count) atomicAdd(&s.mult[ix[e]], 1);
                    lds_barrier();
                    const int times = tid < N ? s.mult[tid] : 0;
                    const uint64_t listed = __ballot(times > 0);
                    if (lane == 0 && wave < 2) s.listed[wave] = listed;
                    lds_barrier();
                    const uint64_t lo = s.listed[0], hi = s.listed[1];
                    auto place = [&](int r) {   // listed rows below r
                        return r < 64 ? __popcll(lo & ((1ull << r) - 1)) : __popcll(lo) + __popcll(hi & ((1ull << (r - 64)) - 1));
                    };
                    if (times > 0) s.bias[place(tid)] = (float)log((double)times);   // exact: see the oracle's log_count
#pragma unroll
                    for (int e = 0; e < 2; ++e)
                        if (ix[e] >= 0 && ix[e] < m.count && cpage_raw[e] >= 0) {
                            const int j = N + place(ix[e]);
                            s.code[j] = cpage_raw[e] * BLOCK_ROWS + ix[e] % BLOCK_ROWS;
                            s.addr[j] = p.cmp + (uint64_t)cpage_raw[e] * p.cmpStride + (uint64_t)((ix[e] % BLOCK_ROWS) * D);
                        }
                }
            }
            lds_barrier();                    // codes visible

            // Tile 0's rows are requested first; the Q encode (staged in tile
            // buffer 1) and the tile loop's per-lane set-up run while they are in
            // flight, then tile 1 follows into the freed buffer.
            issue_tile(0, 0);
            if (first == 0) {
                bool want0 = false, want1 = false;
                for (int i = 0; i < my_tiles; ++i) {
                    const bool kind1 = part + S * i >= m.t0;
                    want0 |= !kind1;
                    want1 |= kind1;
                }
                encode_q(want0, want1);
                lds_barrier();                // every wave holds its Q codes: buffer 1 is free
            }
            if (ntiles > 1) issue_tile(1, 1);

            // The tile loop's per-lane LDS addresses derive from an opaque copy
            // of the lane index, so they are computed here, while the first rows
            // are in flight, rather than ahead of the row codes.
            int lane_x = lane;
            asm volatile("" : "+v"(lane_x));
            const int gx = lane_x >> 4, nx = lane_x & 15;

            // The joint-plan C4 copy holds only the joint route: every live
            // row of such a launch is a joint row (count <= N).
            if (JC4 || joint) {
                // ---- joint row: both tiles resident (tile 0 = window in buffer
                // 0, tile 1 = compressed rows in buffer 1) ----
                vm_wait<0>();
                lds_barrier();
                const int key = 16 * wave + nx;
                const int sl = slot_of(key);
                // QK of both kinds, each with its own Q encoding (reference.py:181-188).
                v4i sacc[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
#pragma unroll
                for (int kind = 0; kind < 2; ++kind) {
                    v4i b[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) b[j] = *reinterpret_cast<const v4i *>(s.tile[kind] + tile_offset(sl, 4 * j + gx));
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        sacc[kind] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kind ? qa1[j] : qa0[j], b[j], sacc[kind], 0, 0, 0);
                }
                float lg[2][2];   // [kind][head 2g + hh]
#pragma unroll
                for (int kind = 0; kind < 2; ++kind) {
                    const bool valid = s.code[kind * N + key] >= 0;
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        float dots = (float)sacc[kind][2 * hh];
                        dots = dots + (float)sacc[kind][2 * hh + 1] * (float)(1.0 / 127.0);
                        float l = dots * s.asc[kind][2 * gx + hh];
                        if (RATIO == 4 && kind == 1) l = l + s.bias[key];   // reference.py:189-190, 261
                        lg[kind][hh] = valid ? l : -1e30f;
                    }
                }
                // maximum = max(sink, every score of both kinds) (reference.py:193)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int kmax = row16_max_key(max(fkey(lg[0][hh]), fkey(lg[1][hh])));
                    if (nx == 0) s.redmax[2 * gx + hh][wave] = kmax;
                }
                lds_barrier();
                float mnew[2], factor[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int h = 2 * gx + hh;
                    const v4i a = *reinterpret_cast<const v4i *>(&s.redmax[h][0]);
                    const v4i b = *reinterpret_cast<const v4i *>(&s.redmax[h][4]);
                    const int k = max(max(max(fkey(mx[hh]), a.x), max(a.y, a.z)), max(max(a.w, b.x), max(max(b.y, b.z), b.w)));
                    mnew[hh] = fkey_value(k);
                }
                {
                    const bool odd = nx & 1;   // exp(sink - maximum), one exponential per lane pair
                    const float mine = sk_expf_nonpos(odd ? mx[1] - mnew[1] : mx[0] - mnew[0]);
                    const float other = dpp<DPP_XOR1>(mine);
                    factor[0] = odd ? other : mine;
                    factor[1] = odd ? mine : other;
                }
                // Weights and P codes (reference.py:194-198); the compressed
                // tile's P codes go to the free address table.
                int8_t *p1 = reinterpret_cast<int8_t *>(s.addr);
                static_assert(16 * PROW <= (int)sizeof(s.addr), "P codes of the second tile fit the address table");
#pragma unroll
                for (int kind = 0; kind < 2; ++kind) {
                    int8_t *pk = kind ? p1 : s.p;
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const float w = sk_expf_nonpos(lg[kind][hh] - mnew[hh]);
                        const float x = w * 127.0f;
                        const float ph = __builtin_rintf(x);
                        const float pl = __builtin_rintf((x - ph) * 127.0f);
                        pk[row_of(2 * gx + hh, 0) * PROW + key] = (int8_t)(int32_t)ph;
                        pk[row_of(2 * gx + hh, 1) * PROW + key] = (int8_t)(int32_t)pl;
                        const float wsum = row16_tree_sum(w);
                        if (nx == 0) (kind ? s.redsum1 : s.redsum)[2 * gx + hh][wave] = wsum;
                    }
                }
                lds_barrier();
                // denominator = exp(sink - maximum) + (window tile's pairwise
                // tree + compressed tile's); zero leaves past a kind's keys
                // change neither tree.
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int h = 2 * gx + hh;
                    const f32x4 a0 = *reinterpret_cast<const f32x4 *>(&s.redsum[h][0]);
                    const f32x4 b0 = *reinterpret_cast<const f32x4 *>(&s.redsum[h][4]);
                    const f32x4 a1 = *reinterpret_cast<const f32x4 *>(&s.redsum1[h][0]);
                    const f32x4 b1 = *reinterpret_cast<const f32x4 *>(&s.redsum1[h][4]);
                    const float t0 = ((a0.x + a0.y) + (a0.z + a0.w)) + ((b0.x + b0.y) + (b0.z + b0.w));
                    const float t1 = ((a1.x + a1.y) + (a1.z + a1.w)) + ((b1.x + b1.y) + (b1.z + b1.w));
                    den[hh] = factor[hh] + (t0 + t1);
                }
                // PV per kind, each added to the output as it completes:
                // output = sum over kinds of dot * (scale / 127) in kind order
                // (reference.py:199-206).
#pragma unroll
                for (int kind = 0; kind < 2; ++kind) {
                    v4i vacc[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) vacc[j] = v4i{0, 0, 0, 0};
                    const lds_i8 *vbase = (const lds_i8 *)(s.tile[kind]);
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb) {
                        const v4i pa = kind ? *reinterpret_cast<const v4i *>(p1 + nx * PROW + 64 * kb + 16 * gx)
                                            : *reinterpret_cast<const v4i *>(s.p + nx * PROW + 64 * kb + 16 * gx);
                        const int sl_lo = slot_of(64 * kb + 16 * gx + (nx >> 1));
                        const int sl_hi = slot_of(64 * kb + 16 * gx + 8 + (nx >> 1));
                        v2i b0[4], b1[4];
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const int chunk = 4 * wave + j;
                            b0[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(vbase + tile_offset(sl_lo, chunk) + 8 * (nx & 1)));
                            b1[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(vbase + tile_offset(sl_hi, chunk) + 8 * (nx & 1)));
                        }
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const v4i vb = {b0[j].x, b0[j].y, b1[j].x, b1[j].y};
                            vacc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vb, vacc[j], 0, 0, 0);
                        }
                    }
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            float dots = (float)vacc[j][2 * hh];
                            dots = dots + (float)vacc[j][2 * hh + 1] * (float)(1.0 / 127.0);
                            const float sc = s.scale[kind][c0 + 16 * j + nx] * (float)(1.0 / 127.0);
                            num[hh][j] = (kind ? num[hh][j] : 0.0f) + dots * sc;   // acc starts at 0
                        }
                    }
                }
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) mx[hh] = mnew[hh];
            } else
            for (int i = 0; i < ntiles; ++i) {
                const int k = part + S * (first + i);
                const int kind = k >= m.t0 ? 1 : 0;
                const int start = (k - (kind ? m.t0 : 0)) * N;
                const int klen = kind ? m.list_len : m.ori_count;
                const int buf = i & 1;
                // Outstanding DMA: tile i, and tile 1 while tile 0 is awaited.
                if (!DEBUG && i == 0 && ntiles > 1) vm_wait<DMA_PER_TILE>();
                else vm_wait<0>();
                lds_barrier();   // every wave's DMA of tile i has landed; every wave is done with tile i - 1
                const bool stream_next = i >= 1 && i + 1 < ntiles;   // tiles 0 and 1 were issued up front
                if (stream_next) issue_rows(i + 1, buf ^ 1, 0, DMA_STEP);
                const int8_t *tb = s.tile[buf];
                const int key = 16 * wave + nx;   // this lane's key in QK and softmax

                // ---- QK: S[16 rows][16 keys of this wave] (reference.py:286-289) ----
                v4i sacc = {0, 0, 0, 0};
                {
                    const int sl = slot_of(key);
                    v4i b[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) b[j] = *reinterpret_cast<const v4i *>(tb + tile_offset(sl, 4 * j + gx));
                    if (kind) {
#pragma unroll
                        for (int j = 0; j < 8; ++j) sacc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa1[j], b[j], sacc, 0, 0, 0);
                    } else {
#pragma unroll
                        for (int j = 0; j < 8; ++j) sacc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa0[j], b[j], sacc, 0, 0, 0);
                    }
                }
                if (stream_next) issue_rows(i + 1, buf ^ 1, DMA_STEP, DMA_STEP);
                if (held) epilogue();            // the previous tile's, behind this tile's QK
                const bool valid = s.code[i * N + key] >= 0;
                float asc[2];
                asc[0] = s.asc[kind][2 * gx];
                asc[1] = s.asc[kind][2 * gx + 1];

                // ---- logits, running max (reference.py:288-303) ----
                float lg[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int32_t hi = sacc[2 * hh], lo = sacc[2 * hh + 1];
                    float dots = (float)hi;
                    dots = dots + (float)lo * (float)(1.0 / 127.0);
                    const float l = dots * asc[hh];
                    lg[hh] = valid ? l : -1e30f;
                    if (DEBUG && dbg.scores && start + key < klen) {
                        // masked rows are zero rows in the reference (reference.py:283-286)
                        int32_t *drow = reinterpret_cast<int32_t *>(dbg.scores) + ((int64_t)t * positions + (kind ? 128 : 0) + start + key) * 16;
                        drow[2 * gx + hh] = valid ? hi : 0;
                        drow[8 + 2 * gx + hh] = valid ? lo : 0;
                    }
                    const int tmax = row16_max_key(fkey(lg[hh]));
                    if (nx == 0) s.redmax[2 * gx + hh][wave] = tmax;
                }
                lds_barrier();
                if (stream_next) issue_rows(i + 1, buf ^ 1, 2 * DMA_STEP, DMA_STEP);
                float mnew[2], factor[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int h = 2 * gx + hh;
                    const v4i a = *reinterpret_cast<const v4i *>(&s.redmax[h][0]);
                    const v4i b = *reinterpret_cast<const v4i *>(&s.redmax[h][4]);
                    const int k = max(max(max(fkey(mx[hh]), a.x), max(a.y, a.z)), max(max(a.w, b.x), max(max(b.y, b.z), b.w)));
                    mnew[hh] = fkey_value(k);
                }
                {
                    // One exponential per lane: even lanes take head 2g, odd lanes
                    // head 2g+1; each lane gets the other head's factor from its
                    // neighbour.
                    const bool odd = nx & 1;
                    const float mine = sk_expf_nonpos(odd ? mx[1] - mnew[1] : mx[0] - mnew[0]);
                    const float other = dpp<DPP_XOR1>(mine);
                    factor[0] = odd ? other : mine;
                    factor[1] = odd ? mine : other;
                }
                // ---- weights, pairwise tile sum, P codes (reference.py:304-312) ----
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const float w = sk_expf_nonpos(lg[hh] - mnew[hh]);
                    const float x = w * 127.0f;
                    const float ph = __builtin_rintf(x);
                    const float pl = resid ? __builtin_rintf((x - ph) * 127.0f) : 0.0f;
                    s.p[row_of(2 * gx + hh, 0) * PROW + key] = (int8_t)(int32_t)ph;
                    s.p[row_of(2 * gx + hh, 1) * PROW + key] = (int8_t)(int32_t)pl;
                    if (DEBUG && dbg.probs && start + key < klen) {
                        int8_t *drow = reinterpret_cast<int8_t *>(dbg.probs) + ((int64_t)t * positions + (kind ? 128 : 0) + start + key) * 16;
                        drow[2 * gx + hh] = (int8_t)(int32_t)ph;
                        drow[8 + 2 * gx + hh] = (int8_t)(int32_t)pl;
                    }
                    const float wsum = row16_tree_sum(w);   // this wave's 16 keys
                    if (nx == 0) s.redsum[2 * gx + hh][wave] = wsum;
                }
                lds_barrier();
                if (stream_next) issue_rows(i + 1, buf ^ 1, 3 * DMA_STEP, DMA_STEP);
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    // Pairwise over the eight 16-key blocks.
                    const int h = 2 * gx + hh;
                    const f32x4 a = *reinterpret_cast<const f32x4 *>(&s.redsum[h][0]);
                    const f32x4 b = *reinterpret_cast<const f32x4 *>(&s.redsum[h][4]);
                    const float tile_sum = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
                    den[hh] = den[hh] * factor[hh] + tile_sum;
                }

                // ---- PV: [16 rows][this wave's 64 columns] (reference.py:310-316) ----
                v4i vacc[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) vacc[j] = v4i{0, 0, 0, 0};
                const lds_i8 *vbase = (const lds_i8 *)(tb);   // generic -> LDS address space
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    // A: P row nx, keys 64 kb + 16 gx .. + 15.  B: two transposed
                    // 8-key reads; lanes 2r / 2r+1 address the two 8-column halves
                    // of key row r, lane nx receives column nx of the 16-column block.
                    const v4i pa = *reinterpret_cast<const v4i *>(s.p + nx * PROW + 64 * kb + 16 * gx);
                    const int sl_lo = slot_of(64 * kb + 16 * gx + (nx >> 1));
                    const int sl_hi = slot_of(64 * kb + 16 * gx + 8 + (nx >> 1));
                    v2i b0[4], b1[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int chunk = 4 * wave + j;
                        b0[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(vbase + tile_offset(sl_lo, chunk) + 8 * (nx & 1)));
                        b1[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(vbase + tile_offset(sl_hi, chunk) + 8 * (nx & 1)));
                    }
                    __builtin_amdgcn_sched_barrier(0);   // all reads in flight before the first MFMA waits
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const v4i vb = {b0[j].x, b0[j].y, b1[j].x, b1[j].y};
                        vacc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vb, vacc[j], 0, 0, 0);
                    }
                }
                if (DEBUG && dbg.values && k < (int)dbg.tileCapacity) {
                    int32_t *vout = reinterpret_cast<int32_t *>(dbg.values) + ((int64_t)t * dbg.tileCapacity + k) * 16 * D;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            vout[(2 * gx + hh) * D + c0 + 16 * j + nx] = vacc[j][2 * hh];
                            vout[(8 + 2 * gx + hh) * D + c0 + 16 * j + nx] = vacc[j][2 * hh + 1];
                        }
                }
                // The FP32 epilogue of this tile runs in the next tile's body,
                // after its QK is issued, so its VALU work overlaps that tile's
                // LDS reads and MFMAs (or after the last tile).
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    held_acc[j] = vacc[j];
                    held_sc[j] = s.scale[kind][c0 + 16 * j + nx];
                }
                held_factor[0] = factor[0];
                held_factor[1] = factor[1];
                held = true;
                mx[0] = mnew[0];
                mx[1] = mnew[1];
            }
            if (first + CODE_TILES < my_tiles) __syncthreads();   // s.code and the tile buffers are rebuilt next
        }
        if (held) epilogue();

        if (folded == 1) {
            // ---- finalize (reference.py:317-323 with one partition) ----
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int h = 2 * g + hh;
                if (ANYH && h >= hlive) continue;
#pragma unroll
                for (int j = 0; j < 4; ++j) out_row[h * D + c0 + 16 * j + n] = (uint16_t)pack_bf16(num[hh][j] / den[hh], 0.0f);
                if (lse_row && wave == 0 && n == 0) lse_row[h] = mx[hh] + logf(den[hh]);
            }
            if (S > 1 && !fused && tid == 0)
                reinterpret_cast<float *>(p.partial)[(int64_t)qrow * S * HEADS * PART_FLOATS + FOLD_SLOT] = 0.0f;
            return;
        }

        // ---- publish this partition: [num 512, max, den] per head ----
        // A fused row whose partitions share this XCD exchanges its states
        // through the XCD's L2 (uniform over the row: a function of the row,
        // the plan and the grid).
        const bool local = (fused & FUSED_XCD_LOCAL) && together;
        float *row_partial = reinterpret_cast<float *>(p.partial) + (int64_t)qrow * S * HEADS * PART_FLOATS;
        const __amdgpu_buffer_rsrc_t states = row_states(row_partial);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int h = 2 * g + hh;
            const int base = ((part * HEADS + h) * PART_FLOATS) * 4;   // byte offset in the row's states
            if (local) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    state_store<SC0>(num[hh][j], states, base + (c0 + 16 * j + n) * 4);
                if (wave == 0 && n == 0) {
                    state_store<SC0>(mx[hh], states, base + 512 * 4);
                    state_store<SC0>(den[hh], states, base + 513 * 4);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    state_store<SC1>(num[hh][j], states, base + (c0 + 16 * j + n) * 4);
                if (wave == 0 && n == 0) {
                    state_store<SC1>(mx[hh], states, base + 512 * 4);
                    state_store<SC1>(den[hh], states, base + 513 * 4);
                }
            }
        }
        if (!fused) {
            if (part == 0 && tid == 0) state_store<SC1>((float)folded, states, FOLD_SLOT * 4);
            return;
        }

        // ---- the last partition of the row to finish folds all of them ----
        // Every state store above has completed (vmcnt 0: acknowledged by
        // the XCD's L2, or by the point of coherence) before the ticket is
        // taken; the partition that takes the last ticket reads the states
        // back with loads of the same scope (sc0 from the shared L2, or sc1).
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        uint32_t *tickets = reinterpret_cast<uint32_t *>(p.workspace);
        if (tid == 0) s.misc[5] = (int)__hip_atomic_fetch_add(&tickets[qrow], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (s.misc[5] != folded - 1) return;
        if (tid == 0) __hip_atomic_store(&tickets[qrow], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        if (local) fold_row<SC0>(states, folded, tid, out_row, lse_row, ANYH ? hlive : HEADS);
        else fold_row<SC1>(states, folded, tid, out_row, lse_row, ANYH ? hlive : HEADS);
    };
    if constexpr (RATIO == 4 && JOINT) {
        if (joint_launch) run_row(std::integral_constant<bool, true>{});
        else run_row(std::integral_constant<bool, false>{});
    } else {
        run_row(std::integral_constant<bool, false>{});
    }
}

// Partition merge as a second launch (merge mode 1): one 512-thread group
// per (query token, group of eight heads), the same fold as the attention
// kernel's last partition, over the partitions that partition 0 recorded.
// Rows it marked 0 (graph padding, or finalized in the attention launch)
// keep what it wrote.
__global__ void __launch_bounds__(THREADS)
c8_merge(const SharedKVArgs p, uint32_t splits)
{
    const int qrow = blockIdx.x, S = (int)splits;
    const int H = (int)p.heads, HG = (H + HEADS - 1) / HEADS;
    const int t = qrow / HG, hbase = HEADS * (qrow % HG);
    float *row_partial = reinterpret_cast<float *>(p.partial) + (int64_t)qrow * S * HEADS * PART_FLOATS;
    const int folded = (int)row_partial[FOLD_SLOT];
    if (folded < 2 || folded > S) return;
    uint16_t *out_row = reinterpret_cast<uint16_t *>(p.out) + ((int64_t)t * H + hbase) * D;
    float *lse_row = p.lse ? reinterpret_cast<float *>(p.lse) + (int64_t)t * H + hbase : nullptr;
    fold_row<0>(row_states(row_partial), folded, threadIdx.x, out_row, lse_row,
                H - hbase < HEADS ? H - hbase : HEADS);
}

// ---- c8_rows: one-partition launches of many query rows ----
// The same numerics as c8_attention with one partition (128-key tiles,
// reference.py:210-323), laid out so that two work-groups share a CU: four
// waves and one tile buffer each (80 KiB of LDS), each work-group taking rows
// r, r + grid, ... in turn.
// When graph padding leaves fewer live rows than the launch's capacity and
// the launch may merge (`fused`: partition states and tickets supplied), the
// live rows are re-planned with c8_attention's PLAN_FEW / PLAN_MANY rule
// (not its one-tile plan for few rows: each partition here repeats the
// row's set-up on four waves, and one-tile partitions measured slower):
// each work item is a (row, partition) pair, every XCD takes a contiguous
// eighth of the live rows, and the last partition of a row folds the
// states.  A row's tiles are a chain (QK -> tile maximum -> exponentials and
// P codes -> PV) through work-group barriers; with one row per CU nothing
// fills those waits, with two rows per CU the other work-group computes
// while this one waits for its barrier or its next tile.  Each wave takes 32 keys in QK (two 16-key blocks) and 128 output
// columns in PV.
// RATIO 4: the window tile and up to eight compressed tiles, every row's HBM
// address resident in LDS.  RATIO 1: the window tile alone.  (C128 launches
// keep c8_attention: its two-tile ring keeps two tiles of a row in flight,
// where this kernel's single buffer exposes one copy round trip per tile; on
// C128 rows of three tiles and on joint rows that costs more than the second
// work-group per CU gains.)
// No explicit original slots.  STREAM: non-temporal KV copies (decode-shaped
// launches).  ANYH: 1..128 heads, a row being one group of eight heads of a
// token (residual codes off above eight heads, reference.py:221-222), as in
// c8_attention.
constexpr int ROWS_THREADS = 256;
constexpr int ROWS_WAVES = ROWS_THREADS / 64;
constexpr int ROWS_TILES = 1 + MAX_LIST / N;                       // a C4 row: window tile + compressed tiles
constexpr int ROWS_DMA = N * D / 1024 / ROWS_WAVES;               // LDS DMA instructions per wave and tile
constexpr int ROWS_IX = MAX_LIST / ROWS_THREADS;                  // C4 index entries per thread
static_assert(ROWS_DMA == 16 && ROWS_IX == 4, "four waves: 32 keys and 16 copies per wave and tile");

struct alignas(16) RowsShared {
    int32_t redmax[HEADS][ROWS_WAVES];   // per-wave maxima of the tile (fkey)
    float redsum[HEADS][ROWS_WAVES];     // per-wave sums of the wave's two 16-key blocks
    float asc[2][HEADS];                 // alpha * softmax_scale per kind
    int32_t scan[ROWS_WAVES];
    int32_t misc[8];
    float scale[2][D];                   // channel scales of the window / compressed cache
    int8_t p[16 * PROW];                 // P codes [MFMA row][key]
    uint64_t addr[ROWS_TILES * N];       // HBM address of each row of the row's tiles (masked: the Q base)
    int8_t tile[N * D];                  // the tile buffer; Q code staging before the first tile
};
static_assert(sizeof(RowsShared) <= 80 * 1024, "two work-groups per CU");
static_assert(offsetof(RowsShared, tile) % 16 == 0, "16-byte LDS DMA rows and tile reads");

template <int RATIO, bool STREAM, bool ANYH>
__global__ void __launch_bounds__(ROWS_THREADS, 2)
c8_rows(const uint64_t cu_q, const uint64_t seq_lens, const uint64_t q_base, const uint64_t cmp_indices,
        const uint32_t batch_arg, const uint32_t topk_arg, const uint32_t rows_arg, const uint32_t grid,
        const uint32_t heads_arg, const SharedKVArgs p, const uint32_t fused)
{
    static_assert(RATIO == 1 || RATIO == 4, "window-only and C4 launches");
    __shared__ RowsShared s;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // scalar: copy destinations on the SALU
    // XCD-aware order: consecutive rows stay on one XCD (their windows overlap).
    const uint32_t G = grid;
    // (Work-groups past the rows still take part: a re-planned launch hands
    // out its items per XCD.)
    const int32_t first_row = (int32_t)((blockIdx.x & 7u) * (G >> 3) + (blockIdx.x >> 3));
    const __attribute__((address_space(1))) int32_t *cu = gptr<int32_t>(cu_q);
    const __attribute__((address_space(1))) int32_t *lens = gptr<int32_t>(seq_lens);
    const int batch_n = (int)batch_arg, topk = RATIO == 4 ? (int)topk_arg : 0;

    // ---- live shape (attention_impl.h:121-137), once per work-group ----
    if (tid == 0) s.misc[0] = 0;
    __syncthreads();
    for (int b = tid; b < batch_n; b += ROWS_THREADS)
        if (lens[b] > 0 && cu[b + 1] >= 0) atomicMax(&s.misc[0], b + 1);
    __syncthreads();
    const int live_batch = uni(s.misc[0]);
    const int end = live_batch ? cu[live_batch] : 0;
    const int live_tokens = end <= 0 ? 0 : (end < (int)p.tokens ? end : (int)p.tokens);
    const int H = ANYH ? (int)heads_arg : HEADS;                 // heads of a query token
    const int HG = ANYH ? (H + HEADS - 1) / HEADS : 1;           // groups of eight
    const bool resid = !ANYH || H <= HEADS;
    // Channel scales: the window's, and the compressed cache's (none without one).
    if (RATIO != 1 || tid < ROWS_THREADS / 2)
        *reinterpret_cast<f32x4 *>(&s.scale[tid >> 7][(tid & 127) * 4]) =
            *gptr<f32x4>(((tid >> 7) ? p.cmpScale : p.oriScale) + (uint64_t)((tid & 127) * 4) * 4);
    const int c0 = 128 * wave;   // this wave's PV output columns: c0 + 16 j + n

    // ---- device plan of a padded launch (c8_attention's rule) ----
    const int32_t rows_cap = (int32_t)rows_arg, live_rows = live_tokens * HG;
    int32_t S = 1;
    const bool replan = fused && live_rows > 0 && live_rows < rows_cap;
    if (replan) {
        if (tid == 0) s.misc[6] = 0;
        __syncthreads();
        for (int b = tid; b < live_batch; b += ROWS_THREADS)
            if (lens[b] > 0 && cu[b + 1] >= 0) atomicMax(&s.misc[6], lens[b]);
        __syncthreads();
        const int longest = uni(s.misc[6]);
        int32_t tiles = 1;
        if (RATIO == 4) {
            const int cnt = longest / 4 < topk ? longest / 4 : topk;
            tiles += (cnt + N - 1) / N;
        }
        int32_t plan = live_rows * PLAN_FEW <= PLAN_CUS ? PLAN_FEW : PLAN_MANY;
        const int32_t fit = PLAN_CUS / live_rows > 1 ? PLAN_CUS / live_rows : 1;
        const int32_t room = rows_cap / live_rows;
        plan = plan < fit ? plan : fit;
        plan = plan < tiles ? plan : tiles;
        plan = plan < room ? plan : room;
        S = plan > 1 ? plan : 1;
        // Padding rows [live_rows, rows_cap) are zero (attention_impl.h:443-460).
        for (int32_t pad = live_rows + first_row; pad < rows_cap; pad += (int32_t)G) {
            const int32_t pt = ANYH ? pad / HG : pad, ph = ANYH ? HEADS * (pad % HG) : 0;
            const int pl = ANYH ? (H - ph < HEADS ? H - ph : HEADS) : HEADS;
            uint16_t *o = reinterpret_cast<uint16_t *>(p.out) + ((int64_t)pt * H + ph) * D;
#pragma unroll
            for (int i = 0; i < 2; ++i)
                if (!ANYH || tid + ROWS_THREADS * i < pl * (D / 8))
                    reinterpret_cast<v4i *>(o)[tid + ROWS_THREADS * i] = v4i{0, 0, 0, 0};
            if (p.lse && tid < pl) reinterpret_cast<float *>(p.lse)[(int64_t)pt * H + ph + tid] = 0.0f;
        }
    }

    // Work item (query row qrow, partition part of S).
    auto run_item = [&](const int32_t qrow, const int32_t part) {
        const int t = ANYH ? qrow / HG : qrow;                   // token
        const int hbase = ANYH ? HEADS * (qrow % HG) : 0;        // first head of the row
        const int hlive = ANYH ? (H - hbase < HEADS ? H - hbase : HEADS) : HEADS;
        uint16_t *out_row = reinterpret_cast<uint16_t *>(p.out) + ((int64_t)t * H + hbase) * D;
        float *lse_row = p.lse ? reinterpret_cast<float *>(p.lse) + (int64_t)t * H + hbase : nullptr;
        // Q (heads wave and wave + 4, channels 8 lane ..) and the row's index
        // entries 4 tid .. 4 tid + 3, requested with the request search (the
        // other work-group of the CU computes meanwhile).
        // Q, the indices and the output are read or written once: non-temporal,
        // so they do not displace the KV rows the launch's rows share in L2.
        v4i qv[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
            qv[hh] = !ANYH || wave + 4 * hh < hlive
                         ? __builtin_nontemporal_load(
                               gptr<v4i>(q_base + (((uint64_t)t * H + hbase + wave + 4 * hh) * D + lane * 8) * 2))
                         : v4i{0, 0, 0, 0};   // padding heads of the last group: zero Q, never written
        int ix[ROWS_IX];
        if (RATIO == 4) {
            const __attribute__((address_space(1))) int32_t *row_ix = gptr<int32_t>(cmp_indices) + (int64_t)t * topk;
#pragma unroll
            for (int e = 0; e < ROWS_IX; ++e)
                ix[e] = tid * ROWS_IX + e < topk ? __builtin_nontemporal_load(row_ix + tid * ROWS_IX + e) : -1;
        }
        __syncthreads();   // every wave is done with the previous item's shared data
        if (tid == 0) s.misc[1] = -1;
        __syncthreads();
        for (int b = tid; b < live_batch; b += ROWS_THREADS) {
            const int b0 = cu[b], b1 = cu[b + 1];
            if (b0 <= t && t < b1) {
                s.misc[1] = b;
                s.misc[3] = lens[b];
                s.misc[4] = b1;
            }
        }
        __syncthreads();
        const int batch = uni(s.misc[1]);
        const int position = batch < 0 ? -1 : uni(s.misc[3]) - uni(s.misc[4]) + t;
        // Padding rows of a captured graph (attention_impl.h:443-460) and rows
        // with a negative position (reference.py:104-105 rejects them) are zero.
        if (t >= live_tokens || batch < 0 || position < 0) {
            if (part != 0) return;
#pragma unroll
            for (int i = 0; i < 2; ++i)
                if (!ANYH || tid + ROWS_THREADS * i < hlive * (D / 8))
                    reinterpret_cast<v4i *>(out_row)[tid + ROWS_THREADS * i] = v4i{0, 0, 0, 0};
            if (lse_row && tid < hlive) lse_row[tid] = 0.0f;
            return;
        }

        // ---- selection (attention_impl.h:58-73, reference.py:228-253) ----
        const int first_ori = position + 1 > WINDOW ? position + 1 - WINDOW : 0;
        const int ori_count = position + 1 - first_ori;
        const int count = RATIO == 4 ? (position + 1) / 4 : 0;
        const __attribute__((address_space(1))) int32_t *otab = gptr<int32_t>(p.oriTable) + (int64_t)batch * p.oriTableWidth;
        const __attribute__((address_space(1))) int32_t *ctab = gptr<int32_t>(p.cmpTable) + (int64_t)batch * p.cmpTableWidth;
        int wpage = -1, widx = -1, cpage[ROWS_IX];
        if (tid < ori_count) {
            const int idx = first_ori + tid;
            if (idx / BLOCK_ROWS < (int)p.oriTableWidth) {
                widx = idx;
                wpage = otab[idx / BLOCK_ROWS];
            }
        }
        int ipos[ROWS_IX];
        int list_len = 0;
        bool ok[ROWS_IX];
        if (RATIO == 4) {
#pragma unroll
            for (int e = 0; e < ROWS_IX; ++e) {
                ok[e] = ix[e] >= 0 && ix[e] < count;
                cpage[e] = ok[e] && ix[e] / BLOCK_ROWS < (int)p.cmpTableWidth ? ctab[ix[e] / BLOCK_ROWS] : -1;
            }
            // List place of each entry: compacted (count < topk <= 1024,
            // reference.py:250) or in place with holes masked.
            list_len = topk;
            if (count < topk) {
                uint64_t v[ROWS_IX];
                int below = 0, mine = 0;
#pragma unroll
                for (int e = 0; e < ROWS_IX; ++e) {
                    v[e] = __ballot(ok[e]);
                    below += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(v[e] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)v[e], 0u));
                    mine += __popcll(v[e]);
                }
                if (lane == 0) s.scan[wave] = mine;
                lds_barrier();
                int at = below, total = 0;
#pragma unroll
                for (int w = 0; w < ROWS_WAVES; ++w) {
                    at += w < wave ? s.scan[w] : 0;
                    total += s.scan[w];
                }
#pragma unroll
                for (int e = 0; e < ROWS_IX; ++e) ipos[e] = ok[e] ? at++ : -1;
                list_len = uni(total);
            } else {
#pragma unroll
                for (int e = 0; e < ROWS_IX; ++e) ipos[e] = ok[e] ? tid * ROWS_IX + e : -1;
            }
        }
        const int tiles = 1 + (list_len + N - 1) / N;   // window tile, then compressed tiles
        // Tile k belongs to partition k % S (the window tile to partition 0);
        // partitions that own no tile hold the initial state, which folds to
        // nothing, and publish nothing.
        if (part >= tiles) return;
        const int folded = S < tiles ? S : tiles;

        // ---- row addresses (masked rows: the Q base, never used) ----
        for (int i = tid; i < tiles * N; i += ROWS_THREADS) s.addr[i] = p.q;
        lds_barrier();
        if (widx >= 0 && wpage >= 0 && (uint32_t)wpage < p.oriPages)
            s.addr[tid] = p.ori + (uint64_t)wpage * p.oriStride + (uint64_t)((widx % BLOCK_ROWS) * D);
        if (RATIO == 4) {
#pragma unroll
            for (int e = 0; e < ROWS_IX; ++e)
                if (ipos[e] >= 0 && cpage[e] >= 0)
                    s.addr[N + ipos[e]] = p.cmp + (uint64_t)cpage[e] * p.cmpStride + (uint64_t)((ix[e] % BLOCK_ROWS) * D);
        }

        // ---- Q folding and residual split per kind (reference.py:274-279) ----
        // Staged in the tile buffer, then picked up in the MFMA A layout.
        v4i qa0[8], qa1[8];
        {
            const int want = (part == 0 ? S : part) < tiles ? 2 : 1;   // a compressed tile in this item
            const int qe0 = lane * 8;
#pragma unroll
            for (int kind = 0; kind < 2; ++kind) {
                if (kind >= want) continue;
                const float *scale = s.scale[kind] + qe0;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int h = wave + 4 * hh;
                    const uint32_t qw[4] = {(uint32_t)qv[hh].x, (uint32_t)qv[hh].y, (uint32_t)qv[hh].z, (uint32_t)qv[hh].w};
                    float f[8];
                    float amax = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        f[e] = bf16_to_f32((qw[e >> 1] >> (16 * (e & 1))) & 0xffffu) * scale[e];
                        amax = fmaxf(amax, fabsf(f[e]));
                    }
                    amax = wave_max(amax);
                    float alpha = amax * (float)(1.0 / 127.0);
                    alpha = alpha < 1e-12f ? 1e-12f : alpha;
                    const float inv = 1.0f / alpha;
                    uint32_t hiw[2] = {0, 0}, low[2] = {0, 0};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float x = clamp127(f[e] * inv);
                        const float hi = __builtin_rintf(x);
                        const float lo = resid ? __builtin_rintf((x - hi) * 127.0f) : 0.0f;
                        hiw[e >> 2] |= ((uint32_t)(int32_t)hi & 0xffu) << (8 * (e & 3));
                        low[e >> 2] |= ((uint32_t)(int32_t)lo & 0xffu) << (8 * (e & 3));
                    }
                    int8_t *stage = s.tile + kind * 16 * QSTAGE;
                    *reinterpret_cast<u32x2 *>(stage + row_of(h, 0) * QSTAGE + qe0) = u32x2{hiw[0], hiw[1]};
                    *reinterpret_cast<u32x2 *>(stage + row_of(h, 1) * QSTAGE + qe0) = u32x2{low[0], low[1]};
                    if (lane == 0) s.asc[kind][h] = alpha * p.softmaxScale;
                }
            }
            lds_barrier();
            const int8_t *st0 = s.tile, *st1 = s.tile + 16 * QSTAGE;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                qa0[jj] = *reinterpret_cast<const v4i *>(st0 + n * QSTAGE + 64 * jj + 16 * g);
                qa1[jj] = want > 1 ? *reinterpret_cast<const v4i *>(st1 + n * QSTAGE + 64 * jj + 16 * g) : v4i{0, 0, 0, 0};
            }
            lds_barrier();   // every wave holds its Q codes: the buffer is free
        }

        // ---- tiles (reference.py:280-316 with one partition) ----
        const __attribute__((address_space(1))) float *sinks = gptr<float>(p.sinks);
        const float den0 = part == 0 ? 1.0f : 0.0f;   // the sink's exp(sink - max) starts partition 0
        float mx[2], den[2] = {den0, den0}, num[2][8];
        mx[0] = (!ANYH || 2 * g < hlive) ? sinks[hbase + 2 * g] : 0.0f;
        mx[1] = (!ANYH || 2 * g + 1 < hlive) ? sinks[hbase + 2 * g + 1] : 0.0f;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int j = 0; j < 8; ++j) num[hh][j] = 0.0f;
        v4i held_acc[8];
        float held_sc[8], held_factor[2];
        bool held = false;
        const uint32_t dst = (uint32_t)(uintptr_t)(lds_i8 *)(s.tile);
        // Tile k with the Q codes of its kind: the window tile (k = 0) takes
        // qa0, whose registers are free for the compressed tiles after it.
        auto run_tile = [&](const int k, const v4i (&qa)[8]) {
            const int kind = k > 0 ? 1 : 0;
            const int lane_x = lane;
            // Copies of tile k: instruction i of wave w moves keys 16 G + r and
            // 16 G + 8 + r (G = 2 w + i / 8, r = i % 8) into slots 16 G + 2 r
            // and 16 G + 2 r + 1, the layout slot_of / tile_offset read.
            {
                const int h = lane_x >> 5, c = lane_x & 31;
                typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int grp = 2 * wave + half;
                    const u64x2 *rows = reinterpret_cast<const u64x2 *>(s.addr + k * N + 16 * grp + 8 * h);
                    u64x2 ra[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) ra[r] = rows[r];
                    const int hx = (h ^ grp) & 1;
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        const int chunk = c ^ r ^ (hx << 3);
                        dma16<STREAM>(ra[r >> 1][r & 1] + (uint32_t)(chunk << 4),
                                      (uint32_t)uni((int)(dst + (16 * grp + 2 * r) * D)));
                    }
                }
            }
            if (held) {
                // The previous tile's FP32 epilogue (reference.py:313-316) while
                // this tile's rows are in flight.
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        float dots = (float)held_acc[j][2 * hh];
                        dots = dots + (float)held_acc[j][2 * hh + 1] * (float)(1.0 / 127.0);
                        const float pv = dots * held_sc[j] * (float)(1.0 / 127.0);
                        num[hh][j] = num[hh][j] * held_factor[hh] + pv;
                    }
            }
            // This wave's copies of tile k have landed.  Its QK keys are the
            // rows it copied itself, so QK needs no barrier; the tile-maximum
            // barrier below makes every wave's rows visible before PV.
            vm_wait<0>();
            // Prefill (rows from L2): the wave in its tile chain issues ahead
            // of the other work-group's wave on the SIMD (copies, epilogue)
            // until the tile ends.  Decode launches, bound by the stream,
            // keep equal priority.
            if (!STREAM) __builtin_amdgcn_s_setprio(1);

            // ---- QK: S[16 rows][32 keys of this wave] (reference.py:286-289) ----
            v4i sacc[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int sl = slot_of(32 * wave + 16 * kb + n);
                v4i b[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) b[j] = *reinterpret_cast<const v4i *>(s.tile + tile_offset(sl, 4 * j + g));
#pragma unroll
                for (int j = 0; j < 8; ++j) sacc[kb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[j], b[j], sacc[kb], 0, 0, 0);
            }
            // ---- logits and the tile maximum (reference.py:288-303) ----
            float lg[2][2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const bool valid = s.addr[k * N + 32 * wave + 16 * kb + n] != p.q;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    float dots = (float)sacc[kb][2 * hh];
                    dots = dots + (float)sacc[kb][2 * hh + 1] * (float)(1.0 / 127.0);
                    const float l = dots * s.asc[kind][2 * g + hh];
                    lg[kb][hh] = valid ? l : -1e30f;
                }
            }
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int kmax = row16_max_key(max(fkey(lg[0][hh]), fkey(lg[1][hh])));
                if (n == 0) s.redmax[2 * g + hh][wave] = kmax;
            }
            lds_barrier();
            float mnew[2], factor[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const v4i a = *reinterpret_cast<const v4i *>(&s.redmax[2 * g + hh][0]);
                mnew[hh] = fkey_value(max(max(fkey(mx[hh]), a.x), max(max(a.y, a.z), a.w)));
            }
            {
                const bool odd = n & 1;   // exp(max_old - max_new), one exponential per lane pair
                const float mine = sk_expf_nonpos(odd ? mx[1] - mnew[1] : mx[0] - mnew[0]);
                const float other = dpp<DPP_XOR1>(mine);
                factor[0] = odd ? other : mine;
                factor[1] = odd ? mine : other;
            }
            // ---- weights, pairwise tile sum, P codes (reference.py:304-312) ----
            float wsum[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                float blk[2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const int key = 32 * wave + 16 * kb + n;
                    const float w = sk_expf_nonpos(lg[kb][hh] - mnew[hh]);
                    const float x = w * 127.0f;
                    const float ph = __builtin_rintf(x);
                    const float pl = resid ? __builtin_rintf((x - ph) * 127.0f) : 0.0f;
                    s.p[row_of(2 * g + hh, 0) * PROW + key] = (int8_t)(int32_t)ph;
                    s.p[row_of(2 * g + hh, 1) * PROW + key] = (int8_t)(int32_t)pl;
                    blk[kb] = row16_tree_sum(w);   // one 16-key block
                }
                wsum[hh] = blk[0] + blk[1];        // blocks 2 w and 2 w + 1
                if (n == 0) s.redsum[2 * g + hh][wave] = wsum[hh];
            }
            lds_barrier();
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const f32x4 a = *reinterpret_cast<const f32x4 *>(&s.redsum[2 * g + hh][0]);
                const float tile_sum = (a.x + a.y) + (a.z + a.w);   // pairwise over the eight blocks
                den[hh] = den[hh] * factor[hh] + tile_sum;
            }
            // ---- PV: [16 rows][this wave's 128 columns] (reference.py:310-316) ----
            v4i vacc[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) vacc[j] = v4i{0, 0, 0, 0};
            const lds_i8 *vbase = (const lds_i8 *)(s.tile);
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const v4i pa = *reinterpret_cast<const v4i *>(s.p + n * PROW + 64 * kb + 16 * g);
                const int sl_lo = slot_of(64 * kb + 16 * g + (n >> 1));
                const int sl_hi = slot_of(64 * kb + 16 * g + 8 + (n >> 1));
#pragma unroll
                for (int jh = 0; jh < 2; ++jh) {
                    v2i b0[4], b1[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int chunk = 8 * wave + 4 * jh + j;
                        b0[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(vbase + tile_offset(sl_lo, chunk) + 8 * (n & 1)));
                        b1[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(vbase + tile_offset(sl_hi, chunk) + 8 * (n & 1)));
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const v4i vb = {b0[j].x, b0[j].y, b1[j].x, b1[j].y};
                        vacc[4 * jh + j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vb, vacc[4 * jh + j], 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                held_acc[j] = vacc[j];
                held_sc[j] = s.scale[kind][c0 + 16 * j + n];
            }
            held_factor[0] = factor[0];
            held_factor[1] = factor[1];
            held = true;
            mx[0] = mnew[0];
            mx[1] = mnew[1];
            if (!STREAM) __builtin_amdgcn_s_setprio(0);
            lds_barrier();   // every wave is done with tile k and the P codes
        };
        // The item's first tile (the window tile on partition 0) takes the Q
        // codes of its kind; the rest are compressed tiles.
        {
            v4i qf[8];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) qf[jj] = part == 0 ? qa0[jj] : qa1[jj];
            run_tile(part, qf);
        }
        for (int k = part + S; k < tiles; k += S) run_tile(k, qa1);
        if (held) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float dots = (float)held_acc[j][2 * hh];
                    dots = dots + (float)held_acc[j][2 * hh + 1] * (float)(1.0 / 127.0);
                    const float pv = dots * held_sc[j] * (float)(1.0 / 127.0);
                    num[hh][j] = num[hh][j] * held_factor[hh] + pv;
                }
        }
        if (folded == 1) {
            // ---- finalize (reference.py:317-323 with one partition) ----
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int h = 2 * g + hh;
                if (ANYH && h >= hlive) continue;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    __builtin_nontemporal_store((uint16_t)pack_bf16(num[hh][j] / den[hh], 0.0f), out_row + h * D + c0 + 16 * j + n);
                if (lse_row && wave == 0 && n == 0) lse_row[h] = mx[hh] + logf(den[hh]);
            }
            return;
        }
        // ---- publish this partition, the last one to finish folds the row
        // (the protocol of c8_attention's fused merge; a re-planned row's
        // partitions all run on one XCD, so with the XCD-local exchange its
        // states pass through that XCD's L2) ----
        const bool local = (fused & FUSED_XCD_LOCAL) != 0;
        const __amdgpu_buffer_rsrc_t states =
            row_states(reinterpret_cast<float *>(p.partial) + (int64_t)qrow * S * HEADS * PART_FLOATS);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int base = ((part * HEADS + 2 * g + hh) * PART_FLOATS) * 4;
            if (local) {
#pragma unroll
                for (int j = 0; j < 8; ++j) state_store<SC0>(num[hh][j], states, base + (c0 + 16 * j + n) * 4);
                if (wave == 0 && n == 0) {
                    state_store<SC0>(mx[hh], states, base + 512 * 4);
                    state_store<SC0>(den[hh], states, base + 513 * 4);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) state_store<SC1>(num[hh][j], states, base + (c0 + 16 * j + n) * 4);
                if (wave == 0 && n == 0) {
                    state_store<SC1>(mx[hh], states, base + 512 * 4);
                    state_store<SC1>(den[hh], states, base + 513 * 4);
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        uint32_t *tickets = reinterpret_cast<uint32_t *>(p.workspace);
        if (tid == 0) s.misc[5] = (int)__hip_atomic_fetch_add(&tickets[qrow], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (s.misc[5] != folded - 1) return;
        if (tid == 0) __hip_atomic_store(&tickets[qrow], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        // fold_row covers eight heads with 512 threads: heads 0-3, then 4-7
        // (one copy of its code: the loop is kept).
#pragma nounroll
        for (int half = 0; half < 2; ++half) {
            if (local) fold_row<SC0>(states, folded, tid + ROWS_THREADS * half, out_row, lse_row, ANYH ? hlive : HEADS);
            else fold_row<SC1>(states, folded, tid + ROWS_THREADS * half, out_row, lse_row, ANYH ? hlive : HEADS);
        }
    };

    // Capacity plan: rows first_row, first_row + G, ...  Re-planned: the live
    // items of this XCD, rows [x R / 8, (x + 1) R / 8) each as S partitions,
    // over the XCD's work-groups in turn.
    const int32_t x = (int32_t)(blockIdx.x & 7u);
    const int32_t lo = replan ? x * live_rows / 8 : 0, hi = replan ? (x + 1) * live_rows / 8 : rows_cap;
    const int32_t step = replan ? (int32_t)(G >> 3) : (int32_t)G;
    for (int32_t j = replan ? (int32_t)(blockIdx.x >> 3) : first_row; lo + j / S < hi; j += step)
        run_item(lo + j / S, j % S);
}

// ---- c8_pairs: query-grouped plans (groups of two or four query tokens) ----
// reference.py:224-323 with query_group G = 2 or 4 (the reference device's
// C128 "paired" and "packed" plans, c128.cpp:17-27): the tokens G j ..
// G j + G - 1 of a request form a group that shares one window list
// (positions max(0, p_first + 1 - 128) .. p_last, up to 127 + G rows) and,
// for C128, one compressed list (rows below (p_last + 1) / 128); each token
// masks what it may not see (its own window, its own compressed count) and
// keeps its own online softmax.  KT-key tiles (KT = 128 or 256, below)
// numbered across both kinds, tile k on partition k % S, no joint rows.  One
// work-group of 8 waves per (sub-pair, partition), a sub-pair being tokens
// 2 i and 2 i + 1 of the request within one group (a group of four has
// two): the group's tiles are fetched into a two-buffer LDS ring (two
// 128-key tiles, or one 256-key tile), waves 0-3 compute the sub-pair's first
// token and waves 4-7 its second, each wave taking 32 keys (64 with 256-key
// tiles) in QK and 128 output columns in PV (the per-row layout of c8_rows).
// Work items are (token, partition); items of the second token of a
// sub-pair exit (the sub-pair's first token takes both), items of padding or
// keyless tokens zero-fill them.  At most eight heads (residual codes on).
// C4 groups (reference.py:242-253 with query_group > 1) list every
// compressed row below (p_last + 1) / 4 once; each token weighs row r by its
// multiplicity m_r among its own valid top-k entries (log(m_r) added to the
// logit, rows with m_r = 0 masked).  The multiplicities of the resident
// tiles are counted in LDS per code chunk (both tokens' counts packed in one
// word), and only rows that one of the two tokens lists are fetched.
// KT = 256: the reference device's grouped plans (c128.cpp:17-27 compile
// them with 256-key tiles; its operator accepts no other tile for grouped
// queries, attention.py:104-106).  A 256-key tile is two 128-row halves, one
// in each buffer of the ring: waves (tok, 0-1) take their QK keys from the
// first half, (tok, 2-3) from the second (64 keys a wave), every wave's PV
// runs over both halves, and the FP32 epilogue runs once per 256 keys.
// With one tile filling the ring, the next tile's copies are issued after
// the current tile's PV.
template <int RATIO, int KT>
struct alignas(16) PairShared {
    // Code slots resident at once (CT 128-row halves' worth).
    static constexpr int CT = RATIO == 4 ? (KT == 256 ? 4 : 8) : CODE_TILES;
    int32_t redmax[2][HEADS][4];   // per token: per-wave tile maxima (fkey)
    float redsum[2][HEADS][4];     // per token: per-wave weight sums of its 16-key blocks
    float asc[2][2][HEADS];        // [token][kind][head]: alpha * softmax_scale
    int32_t misc[8];
    float scale[2][D];             // channel scales of the window / compressed cache
    int8_t p[2][16 * (KT + 16)];   // P codes per token [MFMA row][key]
    int32_t code[CT * N];          // row codes of the resident tiles: page * 32 + row, -1 masked
    uint64_t addr[CT * N];         // HBM address of each resident row (masked rows: the Q base)
    uint32_t mult[RATIO == 4 ? CT * N : 1];   // C4: multiplicity of each resident row, token 0 | token 1 << 16
    float logt[RATIO == 4 ? MAX_LIST + 4 : 1];   // C4: log(m) for multiplicities m = 0 .. MAX_LIST
    alignas(16) int8_t tile[2][N * D];   // the DMA ring; Q code staging before tile 1
};
static_assert(2 * 2 * 16 * QSTAGE <= N * D, "both tokens' Q codes fit one tile buffer");
static_assert(sizeof(PairShared<128, 128>) <= 160 * 1024 && sizeof(PairShared<4, 128>) <= 160 * 1024 &&
                  sizeof(PairShared<128, 256>) <= 160 * 1024 && sizeof(PairShared<4, 256>) <= 160 * 1024,
              "one work-group per CU");
static_assert(2 * MAX_LIST == 4 * THREADS, "four index entries per thread: two tokens' top-k lists");
static_assert(PairShared<4, 256>::CT * N % THREADS == 0 && PairShared<4, 128>::CT * N % THREADS == 0 &&
                  PairShared<128, 128>::CT * N % THREADS == 0 && PairShared<4, 256>::CT * N % 256 == 0,
              "whole code rounds, whole 256-key tiles");
using PairsC4 = PairShared<4, 128>;
using PairsC128 = PairShared<128, 128>;
using PairsC4Wide = PairShared<4, 256>;
using PairsC128Wide = PairShared<128, 256>;
static_assert(offsetof(PairsC4, tile) % 16 == 0 && offsetof(PairsC128, tile) % 16 == 0 &&
                  offsetof(PairsC4Wide, tile) % 16 == 0 && offsetof(PairsC128Wide, tile) % 16 == 0,
              "16-byte LDS DMA rows and tile reads");

template <int RATIO, bool STREAM, int KT>
__global__ void __launch_bounds__(THREADS, 1)
c8_pairs(const uint64_t cu_q, const uint64_t seq_lens, const uint64_t q_base, const uint32_t batch_arg,
         const uint32_t heads_arg, const uint32_t splits, const uint32_t rows_arg, const uint32_t grid,
         const SharedKVArgs p, const uint32_t fused, const uint32_t group)
{
    static_assert(RATIO == 1 || RATIO == 4 || RATIO == 128, "grouped plans: window-only, C4 and C128 launches");
    static_assert(KT == N || KT == 2 * N, "128- or 256-key tiles");
    __shared__ PairShared<RATIO, KT> s;
    constexpr int CT = PairShared<RATIO, KT>::CT;
    constexpr int TPC = CT * N / KT;             // tiles per code chunk
    constexpr int PR = KT + 16;                  // LDS row stride of the P codes
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, n = lane & 15;
    const int tok = wave >> 2, tw = wave & 3;   // token of the group, wave within the token
    const uint32_t G = grid;
    const uint32_t item = (blockIdx.x & 7u) * (G >> 3) + (blockIdx.x >> 3);
    if (item >= rows_arg * splits) return;
    const int S = (int)splits;
    const int t = (int)(item / splits), part = (int)(item % splits);
    const int H = (int)heads_arg;               // 1..8
    const __attribute__((address_space(1))) int32_t *cu = gptr<int32_t>(cu_q);
    const __attribute__((address_space(1))) int32_t *lens = gptr<int32_t>(seq_lens);
    const int batch_n = (int)batch_arg;
    const int mine_b = tid < batch_n ? tid : 0;
    const int my_cu0 = cu[mine_b], my_cu1 = cu[mine_b + 1], my_len = lens[mine_b];
    // Q of both tokens (t and t + 1, which exists when t leads a pair):
    // wave (tok, tw) holds heads tw and tw + 4 of token t + tok, 8 channels
    // per lane.  Rows past the launch read row t instead (never used).
    const int tq = t + tok < (int)rows_arg ? t + tok : t;
    v4i qv[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
        qv[hh] = tw + 4 * hh < H ? *gptr<v4i>(q_base + (((uint64_t)tq * H + tw + 4 * hh) * D + lane * 8) * 2)
                                 : v4i{0, 0, 0, 0};

    // ---- live shape (attention_impl.h:121-137) and the request of token t ----
    if (tid == 0) { s.misc[0] = 0; s.misc[1] = -1; s.misc[2] = 0; }
    __syncthreads();
    for (int b = tid; b < batch_n; b += THREADS) {
        const int len = b == tid ? my_len : lens[b];
        const int c1 = b == tid ? my_cu1 : cu[b + 1];
        if (len > 0 && c1 >= 0) atomicMax(&s.misc[0], b + 1);
    }
    __syncthreads();
    const int live_batch = uni(s.misc[0]);
    for (int b = tid; b < live_batch; b += THREADS) {
        const int c0 = b == tid ? my_cu0 : cu[b];
        const int c1 = b == tid ? my_cu1 : cu[b + 1];
        if (c0 <= t && t < c1) {
            s.misc[1] = b;
            s.misc[3] = b == tid ? my_len : lens[b];
            s.misc[4] = c1;
            s.misc[5] = c0;
        }
        if (b == live_batch - 1) s.misc[2] = c1;
    }
    __syncthreads();
    const int end = live_batch ? uni(s.misc[2]) : 0;
    const int live_tokens = end <= 0 ? 0 : (end < (int)p.tokens ? end : (int)p.tokens);
    const int batch = uni(s.misc[1]);
    uint16_t *out_base = reinterpret_cast<uint16_t *>(p.out);
    float *lse_base = p.lse ? reinterpret_cast<float *>(p.lse) : nullptr;
    auto zero_token = [&](int tz) {   // output and LSE rows of token tz
        if (tid < H * (D / 8)) reinterpret_cast<v4i *>(out_base + (int64_t)tz * H * D)[tid] = v4i{0, 0, 0, 0};
        if (lse_base && tid < H) lse_base[(int64_t)tz * H + tid] = 0.0f;
    };
    // Padding tokens (attention_impl.h:443-460) and tokens of no live request.
    // With a separate merge launch (merge mode 1), partition 0 also marks
    // the tokens it finalizes or zero-fills as having nothing to fold.
    auto no_fold = [&](int tz) {
        if (S > 1 && !fused && tid == 0)
            reinterpret_cast<float *>(p.partial)[(int64_t)tz * S * HEADS * PART_FLOATS + FOLD_SLOT] = 0.0f;
    };
    if (t >= live_tokens || batch < 0) {
        if (part == 0) {
            zero_token(t);
            no_fold(t);
        }
        return;
    }
    const int c0r = uni(s.misc[5]), c1r = uni(s.misc[4]), len = uni(s.misc[3]);
    // Sub-pairs start at even offsets in the request (groups hold an even
    // number of tokens, so no sub-pair straddles two groups).
    if ((t - c0r) & 1) return;                        // the sub-pair's first token takes it
    const int gfirst = c0r + (t - c0r) / (int)group * (int)group;
    int gend = gfirst + (int)group;                   // one past the group's last token
    gend = gend < c1r ? gend : c1r;
    gend = gend < live_tokens ? gend : live_tokens;
    const int gs = t + 1 < gend ? 2 : 1;              // tokens in the sub-pair
    const int p0 = len - c1r + t;                     // position of the sub-pair's first token
    const int pfirst = len - c1r + gfirst, plast = len - c1r + gend - 1;
    if (pfirst < 0) {                                 // negative positions (reference.py:104-105): zero
        if (part == 0) {
            for (int k = 0; k < gs; ++k) {
                zero_token(t + k);
                no_fold(t + k);
            }
        }
        return;
    }
    // ---- the group's lists (reference.py:229-253) ----
    const int lo0 = pfirst + 1 - WINDOW > 0 ? pfirst + 1 - WINDOW : 0;
    const int ori_count = plast + 1 - lo0;            // window rows max(0, pfirst + 1 - 128) .. plast
    const int t0w = (ori_count + KT - 1) / KT;
    const int list_len = RATIO == 1 ? 0 : (plast + 1) / RATIO;   // C4: the group's dense list
    const int total = t0w + (list_len + KT - 1) / KT;
    const int folded = S < total ? S : total;
    if (part >= folded) return;
    const int my_tiles = (total - part + S - 1) / S;
    // Each token's own window and compressed count.
    const int ptok = p0 + (tok < gs ? tok : 0);
    const int own_lo = ptok + 1 - WINDOW > 0 ? ptok + 1 - WINDOW : 0;
    const int own_count = RATIO == 1 ? 0 : (ptok + 1) / RATIO;
    const bool tok_live = tok < gs;
    if (RATIO == 4) {
        // log(m) of every multiplicity a top-k list can give (reference.py:300-301,
        // exact: see the oracle's log_count), read back per key.
        for (int m = tid; m <= MAX_LIST; m += THREADS) s.logt[m] = m > 1 ? (float)log((double)m) : 0.0f;
    }

    const __attribute__((address_space(1))) int32_t *otab = gptr<int32_t>(p.oriTable) + (int64_t)batch * p.oriTableWidth;
    const __attribute__((address_space(1))) int32_t *ctab =
        RATIO != 1 ? gptr<int32_t>(p.cmpTable) + (int64_t)batch * p.cmpTableWidth : otab;
    const __attribute__((address_space(1))) float *sinks = gptr<float>(p.sinks);
    const float sink0 = 2 * g < H ? sinks[2 * g] : 0.0f;
    const float sink1 = 2 * g + 1 < H ? sinks[2 * g + 1] : 0.0f;
    const f32x2 scale_pair = *gptr<f32x2>(((tid >> 8) && RATIO != 1 ? p.cmpScale : p.oriScale) +
                                          (uint64_t)((tid & 255) * 2) * 4);
    const int c0 = 128 * tw;   // this wave's PV output columns: c0 + 16 j + n

    float mx[2] = {sink0, sink1}, den[2], num[2][8];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        den[hh] = part == 0 ? 1.0f : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) num[hh][j] = 0.0f;
    }

    // LDS DMA of resident tile i into ring buffer buf, instructions [r0, r0 + count)
    // of this wave (the layout c8_attention's issue_rows writes).
    auto issue_rows = [&](int i, int buf, int r0, int count) {
        const int h = lane >> 5, c = lane & 31;
        typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
        const u64x2 *rows = reinterpret_cast<const u64x2 *>(s.addr + i * N + 16 * wave + 8 * h + r0);
        u64x2 ra[DMA_PER_TILE / 2];
#pragma unroll
        for (int r = 0; r < DMA_PER_TILE / 2; ++r)
            if (2 * r < count) ra[r] = rows[r];
        const uint32_t dst = (uint32_t)(uintptr_t)(lds_i8 *)(s.tile[buf]) + 16 * wave * D;
        const int hx = (h ^ wave) & 1;
#pragma unroll
        for (int k = 0; k < DMA_PER_TILE; ++k) {
            if (k >= count) break;
            const int r = r0 + k;
            const int chunk = c ^ r ^ (hx << 3);
            dma16<STREAM>(ra[k >> 1][k & 1] + (uint32_t)(chunk << 4), (uint32_t)uni((int)(dst + 2 * r * D)));
        }
    };
    constexpr int DMA_STEP = DMA_PER_TILE / 4;

    v4i qa0[8], qa1[8];
    for (int first = 0; first < my_tiles; first += TPC) {
        const int ntiles = my_tiles - first < TPC ? my_tiles - first : TPC;
        // ---- row codes of partition tiles [first, first + ntiles) ----
        for (int i = tid; i < ntiles * KT; i += THREADS) {
            s.code[i] = -1;
            s.addr[i] = p.q;
            if (RATIO == 4) s.mult[i] = 0;
        }
        if (RATIO == 4) {
            // Multiplicities of the resident compressed rows, from the top-k
            // entries of both tokens (threads 0-255 the first token's, 256-511
            // the second's, four entries each) that are valid for their token
            // (reference.py:243-245: 0 <= index < count).  List place idx is
            // tile t0w + idx / KT, on this partition when that tile is
            // part + S * l, resident when first <= l < first + ntiles.
            const int u = tid >> 8;
            const int ucount = (p0 + u + 1) / 4;
            const __attribute__((address_space(1))) int32_t *row_ix =
                gptr<int32_t>(p.indices) + (int64_t)(t + (u < gs ? u : 0)) * p.topk;
            int cix[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = (tid & 255) + 256 * e;
                cix[e] = u < gs && j < (int)p.topk ? row_ix[j] : -1;
            }
            lds_barrier();                    // the zero fill is complete
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (cix[e] < 0 || cix[e] >= ucount) continue;
                const int k = t0w + cix[e] / KT;
                if (k % S != part) continue;
                const int l = k / S - first;
                if (l >= 0 && l < ntiles) atomicAdd(&s.mult[l * KT + cix[e] % KT], u ? 65536u : 1u);
            }
            lds_barrier();
        }
        constexpr int PER = CT * N / THREADS;
        int tpage[PER], tidx[PER];
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int i = tid + e * THREADS;
            tidx[e] = -1;
            tpage[e] = -1;
            if (i >= ntiles * KT) continue;
            const int k = part + S * (first + i / KT), r = i % KT;
            if (k < t0w) {
                const int j = k * KT + r;     // place in the group's window list
                const int idx = lo0 + j;
                if (j < ori_count && idx / BLOCK_ROWS < (int)p.oriTableWidth) {
                    tidx[e] = idx;
                    tpage[e] = otab[idx / BLOCK_ROWS];
                }
            } else if (RATIO != 1) {
                const int idx = (k - t0w) * KT + r;
                // C4: rows that neither token lists are not fetched.
                if (idx < list_len && idx / BLOCK_ROWS < (int)p.cmpTableWidth && (RATIO != 4 || s.mult[i])) {
                    tidx[e] = idx;
                    tpage[e] = ctab[idx / BLOCK_ROWS];
                }
            }
        }
        if (first == 0) *reinterpret_cast<f32x2 *>(&s.scale[tid >> 8][(tid & 255) * 2]) = scale_pair;
        lds_barrier();                        // the -1 fill is complete before the writes below
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            if (tidx[e] < 0) continue;
            const int i = tid + e * THREADS;
            const bool window = part + S * (first + i / KT) < t0w;
            const bool ok = tpage[e] >= 0 && (!window || (uint32_t)tpage[e] < p.oriPages);
            if (ok) {
                s.code[i] = tpage[e] * BLOCK_ROWS + tidx[e] % BLOCK_ROWS;
                s.addr[i] = (window ? p.ori : p.cmp) + (uint64_t)tpage[e] * (window ? p.oriStride : p.cmpStride) +
                            (uint64_t)((tidx[e] % BLOCK_ROWS) * D);
            }
        }
        lds_barrier();                        // codes visible

        issue_rows(0, 0, 0, DMA_PER_TILE);
        if (first == 0) {
            // ---- Q folding and residual split per token and kind (reference.py:274-279),
            // staged in tile buffer 1, then picked up in the MFMA A layout ----
            // Window tiles are tiles 0 .. t0w - 1 (t0w <= 2, the window list
            // holding at most 131 rows; t0w = 1 with 256-key tiles): this partition
            // holds one when its first tile is one; a compressed one when its
            // last tile is one.
            const bool want[2] = {part < t0w, part + S * (my_tiles - 1) >= t0w};
            int lx = lane;
            asm volatile("" : "+v"(lx));
            const int qe0 = lx * 8;
#pragma unroll
            for (int kind = 0; kind < 2; ++kind) {
                if (!want[kind]) continue;
                const float *scale = s.scale[kind] + qe0;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int h = tw + 4 * hh;
                    const uint32_t qw[4] = {(uint32_t)qv[hh].x, (uint32_t)qv[hh].y, (uint32_t)qv[hh].z, (uint32_t)qv[hh].w};
                    float f[8];
                    float amax = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        f[e] = bf16_to_f32((qw[e >> 1] >> (16 * (e & 1))) & 0xffffu) * scale[e];
                        amax = fmaxf(amax, fabsf(f[e]));
                    }
                    amax = wave_max(amax);
                    float alpha = amax * (float)(1.0 / 127.0);
                    alpha = alpha < 1e-12f ? 1e-12f : alpha;
                    const float inv = 1.0f / alpha;
                    uint32_t hiw[2] = {0, 0}, low[2] = {0, 0};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float x = clamp127(f[e] * inv);
                        const float hi = __builtin_rintf(x);
                        const float lo_ = __builtin_rintf((x - hi) * 127.0f);
                        hiw[e >> 2] |= ((uint32_t)(int32_t)hi & 0xffu) << (8 * (e & 3));
                        low[e >> 2] |= ((uint32_t)(int32_t)lo_ & 0xffu) << (8 * (e & 3));
                    }
                    int8_t *stage = s.tile[1] + (tok * 2 + kind) * 16 * QSTAGE;
                    *reinterpret_cast<u32x2 *>(stage + row_of(h, 0) * QSTAGE + qe0) = u32x2{hiw[0], hiw[1]};
                    *reinterpret_cast<u32x2 *>(stage + row_of(h, 1) * QSTAGE + qe0) = u32x2{low[0], low[1]};
                    if (lane == 0) s.asc[tok][kind][h] = alpha * p.softmaxScale;
                }
            }
            lds_barrier();
            const int8_t *st0 = s.tile[1] + (tok * 2) * 16 * QSTAGE, *st1 = st0 + 16 * QSTAGE;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                qa0[jj] = want[0] ? *reinterpret_cast<const v4i *>(st0 + n * QSTAGE + 64 * jj + 16 * g) : v4i{0, 0, 0, 0};
                qa1[jj] = want[1] ? *reinterpret_cast<const v4i *>(st1 + n * QSTAGE + 64 * jj + 16 * g) : v4i{0, 0, 0, 0};
            }
            lds_barrier();                    // every wave holds its Q codes: buffer 1 is free
        }
        if constexpr (KT == 2 * N) {
            issue_rows(1, 1, 0, DMA_PER_TILE);           // the second half of tile 0
            for (int i = 0; i < ntiles; ++i) {
                const int k = part + S * (first + i);
                const int kind = k >= t0w ? 1 : 0;
                vm_wait<0>();
                lds_barrier();   // both halves of tile i have landed for every wave
                // ---- QK: S[16 rows][64 keys of this wave] (reference.py:286-289),
                // keys 64 tw .. 64 tw + 63 of the tile, in half tw / 2 ----
                const int8_t *tb = s.tile[tw >> 1];
                float lg[4][2];
                int qx = lane;                   // read addresses from a fresh lane copy (not hoisted)
                asm volatile("" : "+v"(qx));
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    const int key = 64 * tw + 16 * kb + n;    // key of the tile
                    const int sl = slot_of(64 * (tw & 1) + 16 * kb + (qx & 15));   // its slot in its half
                    v4i acc = {0, 0, 0, 0};
#pragma unroll
                    for (int jq = 0; jq < 2; ++jq) {
                        v4i b[4];
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            b[j] = *reinterpret_cast<const v4i *>(tb + tile_offset(sl, 4 * (4 * jq + j) + (qx >> 4)));
                        if (kind) {
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa1[4 * jq + j], b[j], acc, 0, 0, 0);
                        } else {
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa0[4 * jq + j], b[j], acc, 0, 0, 0);
                        }
                    }
                    // ---- logits with this token's masks (reference.py:288-303) ----
                    const int idx = kind ? (k - t0w) * KT + key : lo0 + k * KT + key;
                    const int times = RATIO == 4 && kind ? (int)((s.mult[i * KT + key] >> (16 * tok)) & 0xffffu) : 0;
                    const bool mine = RATIO == 4 && kind ? times > 0
                                      : kind ? idx < own_count : (idx >= own_lo && idx <= ptok);
                    const bool valid = tok_live && mine && s.code[i * KT + key] >= 0;
                    const float bias = RATIO == 4 && kind ? s.logt[times] : 0.0f;
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        float dots = (float)acc[2 * hh];
                        dots = dots + (float)acc[2 * hh + 1] * (float)(1.0 / 127.0);
                        float l = dots * s.asc[tok][kind][2 * g + hh];
                        if (RATIO == 4 && kind) l = l + bias;
                        lg[kb][hh] = valid ? l : -1e30f;
                    }
                    // One block's tile reads in flight at a time: hoisting all
                    // four blocks' reads would need 128 more registers.
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int kmax = row16_max_key(max(max(fkey(lg[0][hh]), fkey(lg[1][hh])),
                                                       max(fkey(lg[2][hh]), fkey(lg[3][hh]))));
                    if (n == 0) s.redmax[tok][2 * g + hh][tw] = kmax;
                }
                lds_barrier();
                float mnew[2], factor[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const v4i a = *reinterpret_cast<const v4i *>(&s.redmax[tok][2 * g + hh][0]);
                    mnew[hh] = fkey_value(max(max(fkey(mx[hh]), a.x), max(max(a.y, a.z), a.w)));
                }
                {
                    const bool odd = n & 1;   // exp(max_old - max_new), one exponential per lane pair
                    const float mine = sk_expf_nonpos(odd ? mx[1] - mnew[1] : mx[0] - mnew[0]);
                    const float other = dpp<DPP_XOR1>(mine);
                    factor[0] = odd ? other : mine;
                    factor[1] = odd ? mine : other;
                }
                // ---- weights, pairwise tile sum, P codes (reference.py:304-312):
                // 16-key blocks 4 tw .. 4 tw + 3, pairwise in key order ----
                int8_t *pt = s.p[tok];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    float blk[4];
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb) {
                        const int key = 64 * tw + 16 * kb + n;
                        const float w = sk_expf_nonpos(lg[kb][hh] - mnew[hh]);
                        const float x = w * 127.0f;
                        const float ph = __builtin_rintf(x);
                        const float pl = __builtin_rintf((x - ph) * 127.0f);
                        pt[row_of(2 * g + hh, 0) * PR + key] = (int8_t)(int32_t)ph;
                        pt[row_of(2 * g + hh, 1) * PR + key] = (int8_t)(int32_t)pl;
                        blk[kb] = row16_tree_sum(w);
                    }
                    if (n == 0) s.redsum[tok][2 * g + hh][tw] = (blk[0] + blk[1]) + (blk[2] + blk[3]);
                }
                lds_barrier();
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const f32x4 a = *reinterpret_cast<const f32x4 *>(&s.redsum[tok][2 * g + hh][0]);
                    const float tile_sum = (a.x + a.y) + (a.z + a.w);   // pairwise over the sixteen blocks
                    den[hh] = den[hh] * factor[hh] + tile_sum;
                }
                // ---- PV: [16 rows][this wave's 128 columns] over the 256 keys,
                // in two halves of 64 columns, each with its FP32 epilogue.  The
                // read addresses come from a fresh lane copy: hoisted out of
                // the tile loop, the 64 of them would not fit beside the Q codes ----
                int lx = lane;
                asm volatile("" : "+v"(lx));
                const int ng = lx >> 4, nn = lx & 15;
#pragma unroll
                for (int jh = 0; jh < 2; ++jh) {
                    v4i vacc[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) vacc[j] = v4i{0, 0, 0, 0};
#pragma unroll
                    for (int kc = 0; kc < 4; ++kc) {   // keys 64 kc .. 64 kc + 63, in half kc / 2
                        const lds_i8 *vbase = (const lds_i8 *)(s.tile[kc >> 1]);
                        const v4i pa = *reinterpret_cast<const v4i *>(pt + nn * PR + 64 * kc + 16 * ng);
                        const int sl_lo = slot_of(64 * (kc & 1) + 16 * ng + (nn >> 1));
                        const int sl_hi = slot_of(64 * (kc & 1) + 16 * ng + 8 + (nn >> 1));
                        v2i b0[4], b1[4];
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const int chunk = 8 * tw + 4 * jh + j;
                            b0[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(vbase + tile_offset(sl_lo, chunk) + 8 * (nn & 1)));
                            b1[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(vbase + tile_offset(sl_hi, chunk) + 8 * (nn & 1)));
                        }
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const v4i vb = {b0[j].x, b0[j].y, b1[j].x, b1[j].y};
                            vacc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vb, vacc[j], 0, 0, 0);
                        }
                        __builtin_amdgcn_sched_barrier(0);   // one 64-key chunk's reads in flight at a time
                    }
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            float dots = (float)vacc[j][2 * hh];
                            dots = dots + (float)vacc[j][2 * hh + 1] * (float)(1.0 / 127.0);
                            const float pv = dots * s.scale[kind][c0 + 16 * (4 * jh + j) + n] * (float)(1.0 / 127.0);
                            num[hh][4 * jh + j] = num[hh][4 * jh + j] * factor[hh] + pv;
                        }
                }
                mx[0] = mnew[0];
                mx[1] = mnew[1];
                if (i + 1 < ntiles) {
                    lds_barrier();   // every wave is done with both halves and the P codes
                    issue_rows(2 * (i + 1), 0, 0, DMA_PER_TILE);
                    issue_rows(2 * (i + 1) + 1, 1, 0, DMA_PER_TILE);
                }
            }
        } else {
        if (ntiles > 1) issue_rows(1, 1, 0, DMA_PER_TILE);

        for (int i = 0; i < ntiles; ++i) {
            const int k = part + S * (first + i);
            const int kind = k >= t0w ? 1 : 0;
            const int buf = i & 1;
            if (i == 0 && ntiles > 1) vm_wait<DMA_PER_TILE>();
            else vm_wait<0>();
            lds_barrier();   // tile i has landed for every wave; every wave is done with tile i - 1
            const bool stream_next = i >= 1 && i + 1 < ntiles;
            if (stream_next) issue_rows(i + 1, buf ^ 1, 0, DMA_STEP);
            const int8_t *tb = s.tile[buf];

            // ---- QK: S[16 rows][32 keys of this wave] (reference.py:286-289) ----
            v4i sacc[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int sl = slot_of(32 * tw + 16 * kb + n);
#pragma unroll
                for (int jq = 0; jq < 2; ++jq) {   // 256 channels at a time
                    v4i b[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const v4i *>(tb + tile_offset(sl, 4 * (4 * jq + j) + g));
                    if (kind) {
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            sacc[kb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa1[4 * jq + j], b[j], sacc[kb], 0, 0, 0);
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            sacc[kb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa0[4 * jq + j], b[j], sacc[kb], 0, 0, 0);
                    }
                }
            }
            if (stream_next) issue_rows(i + 1, buf ^ 1, DMA_STEP, DMA_STEP);
            // ---- logits with this token's masks, tile maximum (reference.py:288-303) ----
            float lg[2][2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int key = 32 * tw + 16 * kb + n;
                const int idx = kind ? (k - t0w) * N + key : lo0 + k * N + key;
                // C4: this token's multiplicity of the row; log(m) joins
                // the logit (reference.py:300-301).
                const int times = RATIO == 4 && kind ? (int)((s.mult[i * N + key] >> (16 * tok)) & 0xffffu) : 0;
                const bool mine = RATIO == 4 && kind ? times > 0
                                  : kind ? idx < own_count : (idx >= own_lo && idx <= ptok);
                const bool valid = tok_live && mine && s.code[i * N + key] >= 0;
                const float bias = RATIO == 4 && kind ? s.logt[times] : 0.0f;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    float dots = (float)sacc[kb][2 * hh];
                    dots = dots + (float)sacc[kb][2 * hh + 1] * (float)(1.0 / 127.0);
                    float l = dots * s.asc[tok][kind][2 * g + hh];
                    if (RATIO == 4 && kind) l = l + bias;
                    lg[kb][hh] = valid ? l : -1e30f;
                }
            }
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int kmax = row16_max_key(max(fkey(lg[0][hh]), fkey(lg[1][hh])));
                if (n == 0) s.redmax[tok][2 * g + hh][tw] = kmax;
            }
            lds_barrier();
            if (stream_next) issue_rows(i + 1, buf ^ 1, 2 * DMA_STEP, DMA_STEP);
            float mnew[2], factor[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const v4i a = *reinterpret_cast<const v4i *>(&s.redmax[tok][2 * g + hh][0]);
                mnew[hh] = fkey_value(max(max(fkey(mx[hh]), a.x), max(max(a.y, a.z), a.w)));
            }
            {
                const bool odd = n & 1;   // exp(max_old - max_new), one exponential per lane pair
                const float mine = sk_expf_nonpos(odd ? mx[1] - mnew[1] : mx[0] - mnew[0]);
                const float other = dpp<DPP_XOR1>(mine);
                factor[0] = odd ? other : mine;
                factor[1] = odd ? mine : other;
            }
            // ---- weights, pairwise tile sum, P codes (reference.py:304-312) ----
            int8_t *pt = s.p[tok];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                float blk[2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const int key = 32 * tw + 16 * kb + n;
                    const float w = sk_expf_nonpos(lg[kb][hh] - mnew[hh]);
                    const float x = w * 127.0f;
                    const float ph = __builtin_rintf(x);
                    const float pl = __builtin_rintf((x - ph) * 127.0f);
                    pt[row_of(2 * g + hh, 0) * PR + key] = (int8_t)(int32_t)ph;
                    pt[row_of(2 * g + hh, 1) * PR + key] = (int8_t)(int32_t)pl;
                    blk[kb] = row16_tree_sum(w);   // one 16-key block
                }
                if (n == 0) s.redsum[tok][2 * g + hh][tw] = blk[0] + blk[1];   // blocks 2 tw and 2 tw + 1
            }
            lds_barrier();
            if (stream_next) issue_rows(i + 1, buf ^ 1, 3 * DMA_STEP, DMA_STEP);
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const f32x4 a = *reinterpret_cast<const f32x4 *>(&s.redsum[tok][2 * g + hh][0]);
                const float tile_sum = (a.x + a.y) + (a.z + a.w);   // pairwise over the eight blocks
                den[hh] = den[hh] * factor[hh] + tile_sum;
            }
            // ---- PV: [16 rows][this wave's 128 columns] (reference.py:310-316),
            // in two halves of 64 columns, each followed by its FP32 epilogue
            // (reference.py:313-316): the registers of a deferred epilogue do
            // not fit beside both kinds' Q codes of the wave's token ----
            const lds_i8 *vbase = (const lds_i8 *)(tb);
#pragma unroll
            for (int jh = 0; jh < 2; ++jh) {
                v4i vacc[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) vacc[j] = v4i{0, 0, 0, 0};
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const v4i pa = *reinterpret_cast<const v4i *>(pt + n * PR + 64 * kb + 16 * g);
                    const int sl_lo = slot_of(64 * kb + 16 * g + (n >> 1));
                    const int sl_hi = slot_of(64 * kb + 16 * g + 8 + (n >> 1));
                    v2i b0[4], b1[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int chunk = 8 * tw + 4 * jh + j;
                        b0[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(vbase + tile_offset(sl_lo, chunk) + 8 * (n & 1)));
                        b1[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(vbase + tile_offset(sl_hi, chunk) + 8 * (n & 1)));
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const v4i vb = {b0[j].x, b0[j].y, b1[j].x, b1[j].y};
                        vacc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vb, vacc[j], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        float dots = (float)vacc[j][2 * hh];
                        dots = dots + (float)vacc[j][2 * hh + 1] * (float)(1.0 / 127.0);
                        const float pv = dots * s.scale[kind][c0 + 16 * (4 * jh + j) + n] * (float)(1.0 / 127.0);
                        num[hh][4 * jh + j] = num[hh][4 * jh + j] * factor[hh] + pv;
                    }
            }
            mx[0] = mnew[0];
            mx[1] = mnew[1];
        }
        }
        if (first + TPC < my_tiles) __syncthreads();   // s.code and the tile buffers are rebuilt next
    }
    const int tt = t + tok;   // this wave's token
    uint16_t *out_row = out_base + (int64_t)tt * H * D;
    if (folded == 1) {
        // ---- finalize (reference.py:317-323 with one partition) ----
        if (part == 0 && tok == 0)
            for (int k = 0; k < gs; ++k) no_fold(t + k);
        if (!tok_live) return;
        int lx = lane;                    // head and column from a fresh lane copy (nothing held across the loop)
        asm volatile("" : "+v"(lx));
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int h = 2 * (lx >> 4) + hh;
            if (h >= H) continue;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                out_row[h * D + c0 + 16 * j + (lx & 15)] = (uint16_t)pack_bf16(num[hh][j] / den[hh], 0.0f);
            if (lse_base && tw == 0 && n == 0) lse_base[(int64_t)tt * H + h] = mx[hh] + logf(den[hh]);
        }
        return;
    }
    // ---- publish this partition's state of each token, the last partition
    // of the group to finish folds both (c8_attention's fused merge) ----
    if (tok_live) {
        const __amdgpu_buffer_rsrc_t states =
            row_states(reinterpret_cast<float *>(p.partial) + (int64_t)tt * S * HEADS * PART_FLOATS);
        int lx = lane;                    // head and column from a fresh lane copy (nothing held across the loop)
        asm volatile("" : "+v"(lx));
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int base = ((part * HEADS + 2 * (lx >> 4) + hh) * PART_FLOATS) * 4;
#pragma unroll
            for (int j = 0; j < 8; ++j) state_store<SC1>(num[hh][j], states, base + (c0 + 16 * j + (lx & 15)) * 4);
            if (tw == 0 && (lx & 15) == 0) {
                state_store<SC1>(mx[hh], states, base + 512 * 4);
                state_store<SC1>(den[hh], states, base + 513 * 4);
            }
        }
    }
    if (!fused) {
        if (part == 0 && tid == 0)
            for (int k = 0; k < gs; ++k)
                state_store<SC1>((float)folded,
                                 row_states(reinterpret_cast<float *>(p.partial) + (int64_t)(t + k) * S * HEADS * PART_FLOATS),
                                 FOLD_SLOT * 4);
        return;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t *tickets = reinterpret_cast<uint32_t *>(p.workspace);
    if (tid == 0) s.misc[6] = (int)__hip_atomic_fetch_add(&tickets[t], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s.misc[6] != folded - 1) return;
    if (tid == 0) __hip_atomic_store(&tickets[t], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
#pragma nounroll
    for (int k = 0; k < gs; ++k)
        fold_row<SC1>(row_states(reinterpret_cast<float *>(p.partial) + (int64_t)(t + k) * S * HEADS * PART_FLOATS),
                      folded, tid, out_base + (int64_t)(t + k) * H * D, lse_base ? lse_base + (int64_t)(t + k) * H : nullptr,
                      H);
}

// ---- INT8 cache writer (cache_write.cpp:9-88): one wave per update row ----
template <typename Index, bool Paired>
__global__ void __launch_bounds__(256)
cache_write(const uint64_t updates, const uint64_t inverse_scale, const uint64_t slot_base, const uint64_t update_stride,
            const uint32_t slot_stride, const uint32_t slot_column_stride, const uint32_t tokens, const CacheWriteArgs a)
{
    // The leading arguments (copies of argument-block fields) arrive preloaded
    // in SGPRs, so the row's loads do not wait for a read of the block.
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= tokens) return;
    // The row's values and the inverse scale are requested together with its
    // slot (every row below `tokens` exists), so a row costs one memory round
    // trip; rows the slot rules skip simply drop them.
    const uint64_t src = updates + ((uint64_t)row * update_stride + lane * 8) * 2;
    const uint64_t inv = inverse_scale + (uint64_t)(lane * 8) * 4;
    const v4i x = *gptr<v4i>(src);
    const f32x4 i0 = *gptr<f32x4>(inv);
    const f32x4 i1 = *gptr<f32x4>(inv + 16);
    const __attribute__((address_space(1))) Index *slots = gptr<Index>(slot_base);
    const int64_t first = (int64_t)slots[(uint64_t)row * slot_stride];
    const int64_t second = Paired ? (int64_t)slots[(uint64_t)row * slot_stride + slot_column_stride] : 0;
    asm volatile("" :: "v"(x), "v"(i0), "v"(i1));   // all loads are in flight before the slot is tested
    if (first < 0) return;
    int64_t page, offset;
    if (Paired) {
        page = first;
        offset = second;
    } else {
        page = first / (int64_t)a.pageSize;
        offset = first % (int64_t)a.pageSize;
    }
    if (page >= (int64_t)a.pages || offset < 0 || offset >= (int64_t)a.pageSize) return;
    const uint32_t w[4] = {(uint32_t)x.x, (uint32_t)x.y, (uint32_t)x.z, (uint32_t)x.w};
    const float iv[8] = {i0.x, i0.y, i0.z, i0.w, i1.x, i1.y, i1.z, i1.w};
    uint32_t packed[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float v = bf16_to_f32((w[i >> 1] >> (16 * (i & 1))) & 0xffffu) * iv[i];
        const int32_t code = (int32_t)__builtin_rintf(clamp127(v));   // reference.py:53
        packed[i >> 2] |= ((uint32_t)code & 0xffu) << (8 * (i & 3));
    }
    int8_t *dst = reinterpret_cast<int8_t *>(a.cache) + (uint64_t)page * a.pageStride + (uint64_t)offset * D + lane * 8;
    *reinterpret_cast<u32x2 *>(dst) = u32x2{packed[0], packed[1]};
}

uint32_t head_groups(uint32_t heads) { return (heads + HEADS - 1) / HEADS; }

int check_attention(const SharedKVArgs *a)
{
    if (!a || a->heads == 0 || a->heads > MAX_HEADS || (a->ratio != 1 && a->ratio != 4 && a->ratio != 128) ||
        a->window != WINDOW)
        return 1;
    if (a->oriBlock != BLOCK_ROWS) return 1;
    // Explicit original slots: at most MAX_LIST per row; slot capacity
    // oriPages * 32 stays below 2^31.
    if (a->oriIndices && (a->oriTopk == 0 || a->oriTopk > MAX_LIST || (a->oriIndices & 3) ||
                          (uint64_t)a->oriPages * BLOCK_ROWS >= (1ull << 31)))
        return 1;
    if (!a->q || !a->ori || !a->oriScale || !a->oriTable || !a->cuQ || !a->seqLens || !a->sinks || !a->out)
        return 1;
    if (a->batch == 0 || a->oriPages == 0) return 1;
    if (a->ratio != 1) {
        if (a->cmpBlock != BLOCK_ROWS || !a->cmp || !a->cmpScale || !a->cmpTable) return 1;
        if (a->cmpStride % 16 || a->cmpStride < BLOCK_ROWS * D || ((a->cmp | a->cmpScale) & 15)) return 1;
    }
    if (a->ratio == 4 && (!a->indices || a->topk == 0 || a->topk > MAX_LIST)) return 1;
    if (a->splits == 0 || a->splits > MAX_SPLITS) return 1;
    // Work-groups of the launch (rows x splits, rounded up to 8) fit the grid.
    if ((uint64_t)a->tokens * head_groups(a->heads) * a->splits > 0x7ffffff8ull) return 1;
    if (a->splits > 1 && (!a->partial || !a->workspace)) return 1;
    if (a->oriStride % 16 || a->oriStride < BLOCK_ROWS * D) return 1;
    if ((a->q | a->ori | a->out | a->oriScale) & 15) return 1;
    return 0;
}

// 0: fused (last partition folds), 1: separate merge launch.  A process-wide
// setting (tests and bench.py use it); read once per launch.
std::atomic<int> g_merge_mode{0};

// ---- dispatch probe: which XCD runs which work-group ----
// The XCD-local state exchange (FUSED_XCD_LOCAL) needs work-groups whose
// blockIdx agree modulo 8 to run on one XCD (the hardware hands work-groups
// to the XCDs in turn).  Once per device the library launches a probe grid
// whose work-groups record their XCC_ID and enables the exchange only if
// the XCC_ID depends on blockIdx modulo 8 alone.  The probe writes a
// file-scope array (no allocation) and synchronizes the stream once; it is
// skipped while the stream is being captured (those launches use the
// device-coherent exchange until a later eager launch has probed).
constexpr int PROBE_GROUPS = 1024;
static __device__ uint32_t probe_xcc[PROBE_GROUPS];

__global__ void __launch_bounds__(64) xcd_probe(uint32_t *out)
{
    // Hardware register 20 (XCC_ID), bits 3:0: the XCD running this work-group.
    if (threadIdx.x == 0) out[blockIdx.x] = __builtin_amdgcn_s_getreg(20 | (3 << 11)) & 15u;
}

std::atomic<int> g_xcd_allowed{1};          // sharedkv_c8_set_xcd_local
std::atomic<int> g_xcd_state[64];           // per device: 0 not probed, 1 off, 2 on
std::mutex g_probe_mutex;

bool xcd_local_dispatch(hipStream_t stream, bool may_probe)
{
    if (!g_xcd_allowed.load(std::memory_order_relaxed)) return false;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return false;
    int known = g_xcd_state[device].load(std::memory_order_acquire);
    if (known) return known == 2;
    if (!may_probe) return false;
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &status) != hipSuccess || status != hipStreamCaptureStatusNone) return false;
    std::lock_guard<std::mutex> lock(g_probe_mutex);
    known = g_xcd_state[device].load(std::memory_order_acquire);
    if (known) return known == 2;
    // Relaxed capture mode for this thread: another thread's global-mode
    // capture does not forbid this thread's synchronization.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const bool exchanged = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
    uint32_t *ptr = nullptr;
    uint32_t host[PROBE_GROUPS];
    bool ok = hipGetSymbolAddress(reinterpret_cast<void **>(&ptr), HIP_SYMBOL(probe_xcc)) == hipSuccess;
    if (ok) {
        hipLaunchKernelGGL(xcd_probe, dim3(PROBE_GROUPS), dim3(64), 0, stream, ptr);
        ok = hipGetLastError() == hipSuccess &&
             hipMemcpyAsync(host, ptr, sizeof(host), hipMemcpyDeviceToHost, stream) == hipSuccess &&
             hipStreamSynchronize(stream) == hipSuccess;
    }
    for (int b = 0; ok && b < PROBE_GROUPS; ++b) ok = host[b] == host[b & 7];
    if (exchanged) (void)hipThreadExchangeStreamCaptureMode(&mode);
    g_xcd_state[device].store(ok ? 2 : 1, std::memory_order_release);
    return ok;
}

template <bool DEBUG, bool ANYH>
void launch_variant(hipStream_t stream, const SharedKVArgs *a, const SharedKVDebug &dbg, bool slots, uint32_t grid,
                    uint32_t splits, uint32_t rows, uint32_t fused, bool small_entry)
{
    // Decode-shaped launches stream their KV rows with the non-temporal
    // policy; window-only (ratio 1) launches keep the default.
    const uint32_t per_slot = a->ratio == 4 ? STREAM_TOKENS_C4 : a->ratio == 128 ? STREAM_TOKENS_C128 : 0;
    const bool streamed = !DEBUG && (uint64_t)a->tokens <= (uint64_t)per_slot * a->batch;
    // Joint rows: C128 kernels always carry them.  C4 kernels carry them
    // (and take them when every live row is short) for launches through the
    // small-launch entry, as the reference's sparse_small entry chooses its
    // narrow route from live lengths (c4_small.cpp:10-19), and for launches
    // whose compressed block table names at most one tile of rows per
    // sequence.  Other C4 launches run kernels without them: compiled in,
    // they cost tiled C4 launches about 1 %.
    const bool joint4 = !DEBUG && !slots && a->heads <= HEADS &&
                        (small_entry || (uint64_t)a->cmpTableWidth * BLOCK_ROWS <= (uint64_t)N);
    // One-partition C4 and window-only launches of more rows than CUs
    // (prefill, large decode batches) without explicit slots run two
    // four-wave work-groups per CU taking rows in turn (c8_rows).  C128
    // launches keep one work-group per row: their rows are three or fewer
    // tiles in a prefill chunk, or joint rows, and c8_attention's two-tile
    // ring measured faster on them (C128 prefill chunk 80 against 85 us,
    // joint rows 63 against 110, decode of 512 rows 51 against 72).
    const bool persist = !DEBUG && !slots && splits == 1 && rows > (uint32_t)PLAN_CUS &&
                         (a->ratio == 1 || (a->ratio == 4 && !joint4));
    if (persist) {
        // Two four-wave work-groups per CU (c8_rows), at most one per row, so
        // that every XCD gets its share of the rows.
        const uint32_t g2 = rows < 2u * (uint32_t)PLAN_CUS ? (rows + 7u) & ~7u : 2u * (uint32_t)PLAN_CUS;
        const auto rows_kernel = a->ratio == 1 ? &c8_rows<1, false, ANYH>
                                 : streamed    ? &c8_rows<4, true, ANYH>
                                               : &c8_rows<4, false, ANYH>;
        hipLaunchKernelGGL(rows_kernel, dim3(g2), dim3(ROWS_THREADS), 0, stream, a->cuQ, a->seqLens, a->q, a->indices,
                           a->batch, a->topk, rows, g2, a->heads, *a, fused);
        return;
    }
    decltype(&c8_attention<1, false, false, ANYH, false, false>) kernel =
        slots ? &c8_attention<1, DEBUG, true, ANYH, false, false>
              : &c8_attention<1, DEBUG, false, ANYH, false, false>;
    if (a->ratio == 4 && joint4)
        kernel = streamed ? &c8_attention<4, DEBUG, false, ANYH, !DEBUG, !DEBUG>
                          : &c8_attention<4, DEBUG, false, ANYH, false, !DEBUG>;
    else if (a->ratio == 4)
        kernel = slots ? (streamed ? &c8_attention<4, DEBUG, true, ANYH, !DEBUG, false>
                                   : &c8_attention<4, DEBUG, true, ANYH, false, false>)
                       : (streamed ? &c8_attention<4, DEBUG, false, ANYH, !DEBUG, false>
                                   : &c8_attention<4, DEBUG, false, ANYH, false, false>);
    else if (a->ratio == 128)
        kernel = slots ? (streamed ? &c8_attention<128, DEBUG, true, ANYH, !DEBUG, true>
                                   : &c8_attention<128, DEBUG, true, ANYH, false, true>)
                       : (streamed ? &c8_attention<128, DEBUG, false, ANYH, !DEBUG, true>
                                   : &c8_attention<128, DEBUG, false, ANYH, false, true>);
    // The leading scalar arguments are the ones the first loads need; the
    // build preloads them into SGPRs (-amdgpu-kernarg-preload-count), so
    // those loads do not wait for a read of the argument block.
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(THREADS), 0, stream, a->cuQ, a->seqLens, a->q, a->indices, a->batch,
                       a->topk, a->heads, splits, rows, grid, *a, dbg, fused);
}

template <bool DEBUG>
int launch_attention(hipStream_t stream, const SharedKVArgs *a, const SharedKVDebug *debug, bool small_entry = false,
                     bool may_probe = true)
{
    if (check_attention(a)) return (int)hipErrorInvalidValue;
    if (a->tokens == 0) return (int)hipSuccess;
    const SharedKVDebug dbg = debug ? *debug : SharedKVDebug{0, 0, 0, 0, 0, 0, 0};
    const uint32_t splits = a->splits;
    const uint32_t rows = a->tokens * head_groups(a->heads);
    const uint32_t items = rows * splits;
    // Partition states may be merged inside the launch (merge mode 0) when
    // the launch has several partitions, or has one and supplies partition
    // states and tickets for the device re-plan of a padded launch.
    const bool merge = g_merge_mode.load(std::memory_order_relaxed) == 0 &&
                       (splits > 1 || (a->partial && a->workspace && !DEBUG));
    uint32_t fused = merge ? FUSED_MERGE | (xcd_local_dispatch(stream, may_probe) ? FUSED_XCD_LOCAL : 0u) : 0u;
    // With the XCD-local exchange, a launch of several partitions whose
    // items per XCD (grid / 8) are not a multiple of splits, so that some
    // row's partitions would fall on two XCDs, takes a grid of
    // 8 x splits x ceil(rows / 8): XCD x then holds whole rows
    // [x ceil(rows / 8), (x + 1) ceil(rows / 8)).
    uint32_t grid = (items + 7u) & ~7u;
    if ((fused & FUSED_XCD_LOCAL) && splits > 1 && !DEBUG && (grid / 8u) % splits != 0 &&
        8ull * splits * ((rows + 7u) / 8u) <= 0x7ffffff8ull)
        grid = 8u * splits * ((rows + 7u) / 8u);
    // Debug dumps hold eight heads and one original tile (list places 0..127) per row.
    if (DEBUG && (a->heads != HEADS || (a->oriIndices && a->oriTopk > N))) return (int)hipErrorInvalidValue;
    const bool slots = a->oriIndices != 0;
    if (!DEBUG && a->heads != HEADS)
        launch_variant<false, true>(stream, a, dbg, slots, grid, splits, rows, fused, small_entry);
    else
        launch_variant<DEBUG, false>(stream, a, dbg, slots, grid, splits, rows, fused, small_entry);
    if (splits > 1 && !fused)
        hipLaunchKernelGGL(c8_merge, dim3(rows), dim3(THREADS), 0, stream, *a, splits);
    return (int)hipGetLastError();
}

// Query-grouped launch (groups of `group` = 2 or 4 tokens, c8_pairs, tiles
// of `keys` = 128 or 256 keys): any ratio, at most eight heads, no explicit
// original slots.  The partition plan is the launch's (`splits`); graph
// padding is zero-filled but not re-planned.
int launch_paired(hipStream_t stream, const SharedKVArgs *a, uint32_t group, uint32_t keys)
{
    if (check_attention(a)) return (int)hipErrorInvalidValue;
    if (a->heads > HEADS || a->oriIndices) return (int)hipErrorInvalidValue;
    if ((group != 2 && group != 4) || (keys != N && keys != 2 * N)) return (int)hipErrorInvalidValue;
    if (a->tokens == 0) return (int)hipSuccess;
    const uint32_t splits = a->splits, rows = a->tokens;
    const uint32_t grid = (rows * splits + 7u) & ~7u;
    const uint32_t fused = splits > 1 && g_merge_mode.load(std::memory_order_relaxed) == 0;
    const bool streamed = a->ratio == 128 && a->tokens <= STREAM_TOKENS_C128 * a->batch;
    const auto kernel = keys == N ? (a->ratio == 1 ? &c8_pairs<1, false, N>
                                     : a->ratio == 4 ? &c8_pairs<4, false, N>
                                     : streamed    ? &c8_pairs<128, true, N>
                                                   : &c8_pairs<128, false, N>)
                                  : (a->ratio == 1 ? &c8_pairs<1, false, 2 * N>
                                     : a->ratio == 4 ? &c8_pairs<4, false, 2 * N>
                                     : streamed    ? &c8_pairs<128, true, 2 * N>
                                                   : &c8_pairs<128, false, 2 * N>);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(THREADS), 0, stream, a->cuQ, a->seqLens, a->q, a->batch, a->heads,
                       splits, rows, grid, *a, fused, group);
    if (splits > 1 && !fused)
        hipLaunchKernelGGL(c8_merge, dim3(rows), dim3(THREADS), 0, stream, *a, splits);
    return (int)hipGetLastError();
}

// ---- scratch of the allocation-free entry point ----
// One array per GPU with a fixed layout: the merge tickets (one uint32 per
// row) in the first NOALLOC_TICKET_BYTES, the partition states from there to
// the end.  The two regions never overlap, whatever the row counts of
// successive launches, so a launch's tickets are never left non-zero by an
// earlier launch's states: the loader zero-fills the array and every fused
// launch leaves the tickets it took zero again.  Only launches with more than
// one partition touch the array at all.  Host code never passes the array's
// name to a kernel: its device address is taken once per device with
// hipGetSymbolAddress and kept in g_scratch.
constexpr uint64_t NOALLOC_SCRATCH_BYTES = 16ull << 20;
constexpr uint64_t NOALLOC_TICKET_BYTES = 4096;
constexpr uint64_t NOALLOC_STATE_BYTES = NOALLOC_SCRATCH_BYTES - NOALLOC_TICKET_BYTES;
// Every row of a merging launch holds at least two partition states, so the
// rows whose states fit the state region have their tickets in the ticket
// region.
static_assert(NOALLOC_STATE_BYTES / (2ull * HEADS * PART_FLOATS * 4) * 4 <= NOALLOC_TICKET_BYTES,
              "the ticket region covers every launch whose states fit");
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
void *g_scratch[MAX_DEVICES];

// Device address of the current device's scratch array (looked up on the
// first call on that device).
int scratch_address(void **out)
{
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return (int)e;
    if (device < 0 || device >= MAX_DEVICES) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch[device]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        g_scratch[device] = ptr;
    }
    *out = g_scratch[device];
    return (int)hipSuccess;
}

uint64_t workspace_bytes(uint32_t rows) { return ((uint64_t)rows * 4 + 255) / 256 * 256; }
// Partition states of a launch: rows x splits of them with several
// partitions; with one partition, the states that the device re-plan of a
// padded launch can reach (at most PLAN_CUS row partitions: the plan gives
// live rows x partitions <= PLAN_CUS whenever it gives more than one).
uint64_t partial_bytes(uint32_t rows, uint32_t splits)
{
    const uint64_t state = (uint64_t)HEADS * PART_FLOATS * 4;
    if (splits > 1) return (uint64_t)rows * splits * state;
    return rows > 1 ? (uint64_t)(rows < (uint32_t)PLAN_CUS ? rows : (uint32_t)PLAN_CUS) * state : 0;
}

// Byte offsets of a launch's tickets and partition states in the
// allocation-free scratch array (constant: 0 and NOALLOC_TICKET_BYTES);
// non-zero when the launch does not fit.  One-partition launches always fit:
// only their device re-plan merges, over at most PLAN_CUS row partitions
// (tickets of at most PLAN_CUS rows, partial_bytes(rows, 1) of states).
int noalloc_layout(uint64_t rows, uint32_t splits, uint64_t *tickets, uint64_t *states)
{
    *tickets = 0;
    *states = NOALLOC_TICKET_BYTES;
    if (rows > UINT32_MAX) return 1;
    if (splits <= 1) return 0;
    if (rows * 4 > NOALLOC_TICKET_BYTES || partial_bytes((uint32_t)rows, splits) > NOALLOC_STATE_BYTES) return 1;
    return 0;
}
static_assert(PLAN_CUS * 4 <= NOALLOC_TICKET_BYTES &&
                  (uint64_t)PLAN_CUS * HEADS * PART_FLOATS * 4 <= NOALLOC_STATE_BYTES,
              "a one-partition launch's re-plan fits the allocation-free scratch");

}  // namespace

extern "C" {

int launch_sharedkv_c8_sparse(uint32_t blocks, void *stream, const SharedKVArgs *args)
{
    if (!blocks) return (int)hipSuccess;
    if (!args || args->ratio != 4) return (int)hipErrorInvalidValue;
    return launch_attention<false>(static_cast<hipStream_t>(stream), args, nullptr);
}

int launch_sharedkv_c8_sparse_small(uint32_t blocks, void *stream, const SharedKVArgs *args)
{
    if (!blocks) return (int)hipSuccess;
    if (!args || args->ratio != 4) return (int)hipErrorInvalidValue;
    return launch_attention<false>(static_cast<hipStream_t>(stream), args, nullptr, true);
}

int launch_sharedkv_c8_dense(uint32_t blocks, void *stream, const SharedKVArgs *args)
{
    if (!blocks) return (int)hipSuccess;
    if (!args || (args->ratio != 128 && args->ratio != 1)) return (int)hipErrorInvalidValue;
    return launch_attention<false>(static_cast<hipStream_t>(stream), args, nullptr);
}

int launch_sharedkv_c8_dense_paired(uint32_t blocks, void *stream, const SharedKVArgs *args)
{
    if (!blocks) return (int)hipSuccess;
    if (!args) return (int)hipErrorInvalidValue;
    return launch_paired(static_cast<hipStream_t>(stream), args, 2, 2 * N);
}

int launch_sharedkv_c8_dense_packed(uint32_t blocks, void *stream, const SharedKVArgs *args)
{
    if (!blocks) return (int)hipSuccess;
    if (!args) return (int)hipErrorInvalidValue;
    return launch_paired(static_cast<hipStream_t>(stream), args, 4, 2 * N);
}

int launch_sharedkv_c8_dense_paired_narrow(uint32_t blocks, void *stream, const SharedKVArgs *args)
{
    if (!blocks) return (int)hipSuccess;
    if (!args) return (int)hipErrorInvalidValue;
    return launch_paired(static_cast<hipStream_t>(stream), args, 2, N);
}

int launch_sharedkv_c8_dense_packed_narrow(uint32_t blocks, void *stream, const SharedKVArgs *args)
{
    if (!blocks) return (int)hipSuccess;
    if (!args) return (int)hipErrorInvalidValue;
    return launch_paired(static_cast<hipStream_t>(stream), args, 4, N);
}

int sharedkv_c8_attention_debug(void *stream, const SharedKVArgs *args, const SharedKVDebug *debug)
{
    return launch_attention<true>(static_cast<hipStream_t>(stream), args, debug);
}

int launch_cache_write(uint32_t blocks, void *stream, const CacheWriteArgs *a)
{
    if (!blocks) return (int)hipSuccess;
    if (!a || !a->cache || !a->updates || !a->slots || !a->inverseScale || a->pageSize == 0)
        return (int)hipErrorInvalidValue;
    if (a->updateStride < D || (a->updates & 15) || (a->inverseScale & 15) || (a->updateStride % 8) ||
        (a->pageStride % 8) || (a->cache & 7) || a->pageStride < (uint64_t)a->pageSize * D)
        return (int)hipErrorInvalidValue;
    if (a->pairedSlots && a->slotColumnStride == 0) return (int)hipErrorInvalidValue;
    if (a->slotStride > UINT32_MAX || a->slotColumnStride > UINT32_MAX) return (int)hipErrorInvalidValue;
    if (a->tokens == 0) return (int)hipSuccess;
    const dim3 grid((a->tokens + 3) / 4);
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto kernel = a->int64Slots ? (a->pairedSlots ? &cache_write<int64_t, true> : &cache_write<int64_t, false>)
                                : (a->pairedSlots ? &cache_write<int32_t, true> : &cache_write<int32_t, false>);
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, a->updates, a->inverseScale, a->slots, a->updateStride,
                       (uint32_t)a->slotStride, (uint32_t)a->slotColumnStride, a->tokens, *a);
    return (int)hipGetLastError();
}

uint64_t sharedkv_c8_workspace_bytes(uint32_t rows, uint32_t splits)
{
    (void)splits;
    return workspace_bytes(rows);
}

uint64_t sharedkv_c8_partial_bytes(uint32_t rows, uint32_t splits) { return partial_bytes(rows, splits); }

int launch_sharedkv_c8_noalloc(uint32_t blocks, void *stream, const SharedKVArgs *args)
{
    if (!blocks) return (int)hipSuccess;
    if (!args) return (int)hipErrorInvalidValue;
    if (args->heads == 0 || args->heads > MAX_HEADS || args->splits == 0 || args->splits > MAX_SPLITS)
        return (int)hipErrorInvalidValue;
    const uint64_t rows = (uint64_t)args->tokens * head_groups(args->heads);
    uint64_t tickets = 0, states = 0;
    if (noalloc_layout(rows, args->splits, &tickets, &states)) return (int)hipErrorInvalidValue;
    void *base = nullptr;
    const int e = scratch_address(&base);
    if (e) return e;
    SharedKVArgs a = *args;
    a.workspace = (uint64_t)(uintptr_t)base + tickets;
    a.partial = (uint64_t)(uintptr_t)base + states;
    // The entry the package routes the launch to: C4 launches of fewer than
    // SMALL_TOKENS tokens as launch_sharedkv_c8_sparse_small.
    // No dispatch probe from here (it copies to the host): the XCD-local
    // exchange applies once another entry has probed this device.
    return launch_attention<false>(static_cast<hipStream_t>(stream), &a, nullptr,
                                   a.ratio == 4 && a.tokens < SMALL_TOKENS, false);
}

uint64_t sharedkv_c8_noalloc_scratch_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

int sharedkv_c8_noalloc_layout(uint32_t rows, uint32_t splits, uint64_t *tickets_offset, uint64_t *states_offset)
{
    if (!tickets_offset || !states_offset || splits == 0 || splits > MAX_SPLITS) return (int)hipErrorInvalidValue;
    return noalloc_layout(rows, splits, tickets_offset, states_offset) ? (int)hipErrorInvalidValue : (int)hipSuccess;
}

int sharedkv_c8_set_merge_mode(int mode)
{
    if (mode != 0 && mode != 1) return (int)hipErrorInvalidValue;
    g_merge_mode.store(mode, std::memory_order_relaxed);
    return (int)hipSuccess;
}

int sharedkv_c8_set_xcd_local(int enable)
{
    if (enable != 0 && enable != 1) return (int)hipErrorInvalidValue;
    g_xcd_allowed.store(enable, std::memory_order_relaxed);
    return (int)hipSuccess;
}

int sharedkv_c8_xcd_local(void)
{
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return -1;
    const int known = g_xcd_state[device].load(std::memory_order_acquire);
    return known == 0 ? -1 : known == 2 ? 1 : 0;
}

uint32_t sharedkv_attention_args_size(void) { return (uint32_t)sizeof(SharedKVArgs); }
uint32_t sharedkv_cache_args_size(void) { return (uint32_t)sizeof(CacheWriteArgs); }
uint32_t sharedkv_abi_version(void) { return 3; }

}  // extern "C"
