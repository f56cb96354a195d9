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
// Design (one GPU, HBM bound).  One work-group of 4 waves per (query row, KV
// partition); partition `part` owns tiles part, part + S, ... of the row's key
// list (window rows, then compressed rows, cut into 128-key tiles).
//   prologue   every independent load of the row (metadata, indices, Q, both
//              scale vectors) is issued at once: one memory round trip
//   addresses  the partition's rows are turned into page codes
//              (page * 32 + row in page, -1 = masked) in LDS: one round trip
//              of block-table reads per chunk of tiles
//   tiles      each of the 4 waves loads its 32 keys straight into the
//              B-operand registers of v_mfma_i32_16x16x64_i8 (QK needs no
//              LDS), writes them once to LDS as the V tile, and issues the
//              next tile's loads into the same registers while softmax and
//              PV run; PV reads V transposed with ds_read_b64_tr_b8.  Two
//              work-groups per CU (256 VGPRs, 80 KB LDS)
//   softmax    FP32 in registers; rows are 8 heads x {code, residual} = the
//              16 MFMA rows; max and pairwise sums cross waves through LDS
//   partials   with S > 1 partitions, FP32 [num, max, den] go to `partial`;
//              the last partition of a row to finish (a ticket per row in
//              `workspace`) folds them, or c8_merge does in a second launch
// Integer partials are exact, so any assignment of keys to lanes gives the
// reference's integers; the FP32 sequence below is kept in the reference's
// order with contraction disabled.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sharedkv_hip.h"

#pragma clang fp contract(off)

namespace {

constexpr int D = 512;
constexpr int HEADS = 8;
constexpr int N = SHAREDKV_C8_TILE;    // keys per tile
constexpr int THREADS = 256;           // 4 waves
constexpr int WAVES = THREADS / 64;
constexpr int VROW = D + 16;           // LDS row stride of the V tile
constexpr int VTILE = N * VROW + (N / 16) * 128;   // each 16-row block adds 128 B
constexpr int PROW = N + 16;           // LDS row stride of the P codes
constexpr int CODE_TILES = 10;         // tiles whose row codes are resident at once
constexpr int MAX_LIST = 1024;         // C4 top-k capacity of the index list
constexpr int PART_FLOATS = 520;       // per (row, split, head): 512 numerator, max, denominator
constexpr int WINDOW = 128;
constexpr int BLOCK_ROWS = 32;
constexpr uint32_t MAX_SPLITS = 16;
static_assert(N == 128 && WINDOW == N, "one window tile of 128 keys; 4 waves x 32 keys");

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
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

// Round to nearest even (torch's .bfloat16()).
__device__ __forceinline__ uint32_t f32_to_bf16(float x)
{
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// exp(x): Cody & Waite reduction x = n ln2 + r with a 16-bit head of ln2 and
// its tail, then the degree-8 Taylor series of e^r in Horner form with fma,
// scaled by 2^n.  The CPU checker evaluates the identical sequence, so the
// softmax weights (and the INT8 P codes derived from them) agree bit for bit.
__device__ __forceinline__ float sk_expf(float x)
{
    if (!(x >= -87.0f)) return x != x ? x : 0.0f;
    if (x > 88.0f) return __builtin_inff();
    float n = __builtin_rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, x);
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
    return __builtin_ldexpf(p, (int)n);
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

// A value that is the same in every lane (read from LDS after a barrier),
// moved to a scalar register so it does not occupy a VGPR.
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }

// LDS byte offset of key row `key` in the V tile.  Rows are 528 B apart and
// each 16-row block starts 128 B further on, so 16-byte row writes of 16
// consecutive keys hit distinct banks (4 banks apart) and the transposed
// 8-row reads of two neighbouring 16-row blocks land on opposite bank halves.
__device__ __forceinline__ int vrow(int key) { return key * VROW + (key >> 4) * 128; }

// MFMA row m of the 16-row operands: rows 4g..4g+3 hold heads 2g and 2g+1,
// each as {code, residual}.  Output lane group g then owns both rows of both
// of its heads.
__device__ __forceinline__ int row_of(int head, int residual) { return 4 * (head >> 1) + 2 * (head & 1) + residual; }

struct Shared {
    int8_t v[VTILE];                // V tile; Q code staging [16][512] at kind switches
    int8_t p[16 * PROW];            // P codes [MFMA row][key]
    int32_t code[CODE_TILES * N];   // row codes of the resident tiles: page * 32 + row, -1 masked
    float scale[2][D];              // channel scales of the window / compressed cache
    float red[2][WAVES][HEADS];     // per-wave max / sum exchange
    float asc[HEADS];               // alpha * softmax_scale of the current kind
    int32_t scan[WAVES];
    int32_t misc[8];
};

struct Row {
    int32_t batch, position, first_ori, ori_count, count, list_len, t0, total;
};

// Partition states are exchanged between work-groups that may sit on
// different XCDs (each with its own L2).  They are written and read with
// buffer accesses carrying the sc1 cache policy (device-coherent: written
// through to, and read from, the point of coherence of all XCDs) instead of
// flushing and invalidating the whole L2 around a device-scope fence.
constexpr int SC1 = 16;                    // cache-policy operand: sc1
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
// Thread = (head tid / 32, columns 16 (tid % 32) .. + 15) of a 256-thread
// group.  Partitions are folded in order.  MAXS bounds S at compile time so
// every load is issued before any is used (offsets of partitions past S are
// clamped to partition 0 and their values ignored).  Returns false, writing
// nothing, for a row partition 0 marked as graph padding (denominator < 0).
template <int MAXS, int POLICY>
__device__ __forceinline__ bool fold_states(const __amdgpu_buffer_rsrc_t states, int S, int tid,
                                            uint16_t *out_row, float *lse_row)
{
    const int h = tid >> 5, col = (tid & 31) * 16;
    const int head_base = h * PART_FLOATS * 4;
    const int part_step = HEADS * PART_FLOATS * 4;
    float ms[MAXS], ds[MAXS];
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) {
        const int at = head_base + (sp < S ? sp : 0) * part_step;
        ms[sp] = state_load<POLICY>(states, at + 512 * 4);
        ds[sp] = state_load<POLICY>(states, at + 513 * 4);
    }
    if (ds[0] < 0.0f) return false;
    float top = ms[0];
#pragma unroll
    for (int sp = 1; sp < MAXS; ++sp) top = sp < S ? fmaxf(top, ms[sp]) : top;
    float f[MAXS], dsum = 0.0f;
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) {
        f[sp] = sk_expf(ms[sp] - top);
        dsum = sp < S ? dsum + ds[sp] * f[sp] : dsum;
    }
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
        f32x4 v[MAXS];
#pragma unroll
        for (int sp = 0; sp < MAXS; ++sp)
            v[sp] = state_load4<POLICY>(states, head_base + (sp < S ? sp : 0) * part_step + (col + 4 * c4) * 4);
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int sp = 0; sp < MAXS; ++sp)
            if (sp < S) {
                acc.x = acc.x + v[sp].x * f[sp];
                acc.y = acc.y + v[sp].y * f[sp];
                acc.z = acc.z + v[sp].z * f[sp];
                acc.w = acc.w + v[sp].w * f[sp];
            }
        const uint32_t lo = f32_to_bf16(acc.x / dsum) | (f32_to_bf16(acc.y / dsum) << 16);
        const uint32_t hi = f32_to_bf16(acc.z / dsum) | (f32_to_bf16(acc.w / dsum) << 16);
        *reinterpret_cast<u32x2 *>(out_row + h * D + col + 4 * c4) = u32x2{lo, hi};
    }
    if (lse_row && (tid & 31) == 0) lse_row[h] = top + logf(dsum);
    return true;
}

template <int POLICY>
__device__ __forceinline__ void fold_row(const __amdgpu_buffer_rsrc_t states, int S, int tid, uint16_t *out_row,
                                         float *lse_row)
{
    if (S <= 4) fold_states<4, POLICY>(states, S, tid, out_row, lse_row);
    else if (S <= 8) fold_states<8, POLICY>(states, S, tid, out_row, lse_row);
    else fold_states<16, POLICY>(states, S, tid, out_row, lse_row);
}

template <int RATIO, bool DEBUG>
__global__ void __launch_bounds__(THREADS, 2)   // 2 waves per SIMD: two work-groups per CU
c8_attention(const SharedKVArgs p, const SharedKVDebug dbg, uint32_t splits, uint32_t items, uint32_t fused)
{
    __shared__ Shared s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, n = lane & 15;

    // XCD-aware order: consecutive work items (the partitions of one row,
    // then the next row) stay on one XCD and share its L2.
    const uint32_t G = gridDim.x;
    const uint32_t item = (blockIdx.x & 7u) * (G >> 3) + (blockIdx.x >> 3);
    if (item >= items) return;
    const int32_t t = (int32_t)(item / splits);
    const int32_t part = (int32_t)(item % splits);
    const int32_t S = (int32_t)splits;

    // ---- prologue: every load that depends only on t, issued together ----
    const int32_t *cu = reinterpret_cast<const int32_t *>(p.cuQ);
    const int32_t *lens = reinterpret_cast<const int32_t *>(p.seqLens);
    const int batch_n = (int)p.batch;
    // Request b's (cu[b], cu[b+1], len[b]) for b = tid (more in the loops below).
    int my_cu0 = 0, my_cu1 = -1, my_len = 0;
    if (tid < batch_n) {
        my_cu0 = cu[tid];
        my_cu1 = cu[tid + 1];
        my_len = lens[tid];
    }
    // Q row t: 8 heads x 512 BF16; thread = head tid / 32, channels (tid % 32) * 16.
    const int qh = tid >> 5, qd0 = (tid & 31) * 16;
    const uint16_t *qrow = reinterpret_cast<const uint16_t *>(p.q) + ((int64_t)t * HEADS + qh) * D + qd0;
    const v4i q0 = *reinterpret_cast<const v4i *>(qrow);
    const v4i q1 = *reinterpret_cast<const v4i *>(qrow + 8);
    // Scales of both kinds into LDS (kind = tid / 128, 4 channels per thread).
    {
        const int kind = tid >> 7, c = (tid & 127) * 4;
        const uint64_t base = (kind && RATIO != 1) ? p.cmpScale : p.oriScale;
        *reinterpret_cast<f32x4 *>(&s.scale[kind][c]) = *gptr<f32x4>(base + (uint64_t)c * 4);
    }
    // C4 index entries 4 tid .. 4 tid + 3 of row t.
    int ix[4] = {-1, -1, -1, -1};
    if (RATIO == 4) {
        const int topk = (int)p.topk;
        const int32_t *row_ix = reinterpret_cast<const int32_t *>(p.indices) + (int64_t)t * topk;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (tid * 4 + i < topk) ix[i] = row_ix[tid * 4 + i];
    }
    const float *sinks = reinterpret_cast<const float *>(p.sinks);
    const float sink0 = sinks[2 * g], sink1 = sinks[2 * g + 1];

    // ---- live shape (attention_impl.h:121-137) and the row's request ----
    if (tid == 0) { s.misc[0] = 0; s.misc[1] = -1; s.misc[2] = 0; }
    __syncthreads();
    for (int b = tid; b < batch_n; b += THREADS) {
        const int len = b == tid ? my_len : lens[b];
        const int c1 = b == tid ? my_cu1 : cu[b + 1];
        if (len > 0 && c1 >= 0) atomicMax(&s.misc[0], b + 1);
    }
    __syncthreads();
    const int live_batch = uni(s.misc[0]);
    for (int b = tid; b < batch_n; b += THREADS) {
        const int c0 = b == tid ? my_cu0 : cu[b];
        const int c1 = b == tid ? my_cu1 : cu[b + 1];
        const int len = b == tid ? my_len : lens[b];
        if (b == live_batch - 1) s.misc[2] = c1;
        if (b < live_batch && c0 <= t && t < c1) {
            s.misc[1] = b;
            s.misc[3] = len;
            s.misc[4] = c1;
        }
    }
    __syncthreads();
    const int end = live_batch ? uni(s.misc[2]) : 0;
    const int live_tokens = end <= 0 ? 0 : (end < (int)p.tokens ? end : (int)p.tokens);
    const int batch = uni(s.misc[1]);
    uint16_t *out_row = reinterpret_cast<uint16_t *>(p.out) + (int64_t)t * HEADS * D;
    float *lse_row = p.lse ? reinterpret_cast<float *>(p.lse) + (int64_t)t * HEADS : nullptr;
    if (t >= live_tokens || batch < 0) {
        // Graph padding rows are zero-filled (attention_impl.h:443-460); with
        // a separate merge launch, partition 0 also marks the row
        // (denominator -1) so that launch leaves it alone.
        if (part == 0) {
            reinterpret_cast<v4i *>(out_row)[tid * 2] = v4i{0, 0, 0, 0};
            reinterpret_cast<v4i *>(out_row)[tid * 2 + 1] = v4i{0, 0, 0, 0};
            if (lse_row && tid < HEADS) lse_row[tid] = 0.0f;
            if (S > 1 && !fused && tid < HEADS)
                reinterpret_cast<float *>(p.partial)[((int64_t)t * S * HEADS + tid) * PART_FLOATS + 513] = -1.0f;
        }
        return;
    }

    // ---- selection (attention_impl.h:58-73, reference.py:228-253) ----
    Row m;
    m.batch = batch;
    m.position = uni(s.misc[3]) - uni(s.misc[4]) + t;
    m.first_ori = m.position + 1 > WINDOW ? m.position + 1 - WINDOW : 0;
    m.ori_count = m.position + 1 - m.first_ori;
    if (m.ori_count < 0) m.ori_count = 0;
    m.count = RATIO == 1 ? 0 : (m.position + 1) / RATIO;
    int ipos[4] = {-1, -1, -1, -1};   // list position of each owned C4 entry (-1: none)
    if (RATIO == 4) {
        const int topk = (int)p.topk;
        const bool compact = m.count < topk && topk <= MAX_LIST;   // reference.py:250
        int ok[4], mine = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ok[i] = ix[i] >= 0 && ix[i] < m.count;
            mine += ok[i];
        }
        if (compact) {
            int incl = mine;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(incl, o);
                if (lane >= o) incl += y;
            }
            if (lane == 63) s.scan[wave] = incl;
            __syncthreads();
            int at = incl - mine, total = 0;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                at += w < wave ? s.scan[w] : 0;
                total += s.scan[w];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (ok[i]) ipos[i] = at++;
            m.list_len = uni(total);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = tid * 4 + i;
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
    const int my_tiles = m.total > part ? (m.total - part + S - 1) / S : 0;   // tiles part, part + S, ...

    // ---- per-lane softmax state for heads 2g and 2g+1 ----
    float mx[2] = {sink0, sink1}, den[2], num[2][8];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        den[hh] = part == 0 ? 1.0f : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) num[hh][j] = 0.0f;
    }

    const int positions = 128 + (int)dbg.cmpCapacity;
    const int c0 = 128 * wave;      // this wave's 128 PV output columns: c0 + 16 j + n

    // Row codes of partition tiles [first, first + CODE_TILES) into s.code.
    auto build_codes = [&](int first) {
        const int ntiles = my_tiles - first < CODE_TILES ? my_tiles - first : CODE_TILES;
        for (int i = tid; i < ntiles * N; i += THREADS) s.code[i] = -1;
        __syncthreads();
        const int32_t *otab = reinterpret_cast<const int32_t *>(p.oriTable) + (int64_t)m.batch * p.oriTableWidth;
        const int32_t *ctab = reinterpret_cast<const int32_t *>(p.cmpTable) + (int64_t)m.batch * p.cmpTableWidth;
        // Rows whose logical page lies outside the block table, or whose
        // physical page is negative or (window cache) past the pool, stay
        // masked instead of being dereferenced.
        for (int i = tid; i < ntiles * N; i += THREADS) {
            const int k = part + S * (first + i / N), r = i % N;
            int idx = -1;
            const int32_t *tab = otab;
            int width = (int)p.oriTableWidth;
            if (k < m.t0) {
                if (r < m.ori_count) idx = m.first_ori + r;
            } else if (RATIO == 128) {
                const int pos = (k - m.t0) * N + r;
                if (pos < m.list_len) idx = pos;
                tab = ctab;
                width = (int)p.cmpTableWidth;
            }
            if (idx >= 0 && idx / BLOCK_ROWS < width) {
                const int32_t page = tab[idx / BLOCK_ROWS];
                const bool ok = page >= 0 && (k >= m.t0 || (uint32_t)page < p.oriPages);
                if (ok) s.code[i] = page * BLOCK_ROWS + idx % BLOCK_ROWS;
            }
        }
        if (RATIO == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (ipos[e] < 0 || ix[e] < 0) continue;
                const int k = m.t0 + ipos[e] / N;
                if (k < part || (k - part) % S) continue;
                const int i = (k - part) / S - first;
                if (i < 0 || i >= ntiles) continue;
                const int idx = ix[e];
                if (idx / BLOCK_ROWS < (int)p.cmpTableWidth) {
                    const int32_t page = ctab[idx / BLOCK_ROWS];
                    if (page >= 0) s.code[i * N + ipos[e] % N] = page * BLOCK_ROWS + idx % BLOCK_ROWS;
                }
            }
        }
        __syncthreads();
    };

    // K rows of resident tile `slot` into the B-operand registers:
    // kq[8 kb + j] = bytes 64 j + 16 g .. + 15 of key 32 wave + 16 kb + n.
    v4i kq[16];
    auto load_tile = [&](int slot, int kind) {
        const uint64_t base = kind ? p.cmp : p.ori;
        const uint64_t stride = kind ? p.cmpStride : p.oriStride;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int code = s.code[slot * N + 32 * wave + 16 * kb + n];
            const uint64_t a = base + (uint64_t)(code >> 5) * stride + (uint64_t)(code & 31) * D + 16 * g;
#pragma unroll
            for (int j = 0; j < 8; ++j) kq[8 * kb + j] = code >= 0 ? *gptr<v4i>(a + 64 * j) : v4i{0, 0, 0, 0};
        }
    };

    v4i qa[8];            // Q codes as MFMA A operands, per 64-byte D block
    float asc[2] = {0.0f, 0.0f};
    float sc[8];          // channel scale of this lane's output columns
    int cur_kind = -1;
    const uint32_t qw[8] = {(uint32_t)q0.x, (uint32_t)q0.y, (uint32_t)q0.z, (uint32_t)q0.w,
                            (uint32_t)q1.x, (uint32_t)q1.y, (uint32_t)q1.z, (uint32_t)q1.w};

    // Q folding and residual split for cache kind `kind` (reference.py:274-279).
    // Runs while no tile is in registers: before the first tile and at the
    // one switch from the window tile to compressed tiles.
    auto encode_q = [&](int kind) {
        const float *scale = s.scale[kind];
        // The packed BF16 words stay packed until here (an opaque copy keeps
        // the compiler from hoisting eight expanded floats out of the loop).
        uint32_t w[8] = {qw[0], qw[1], qw[2], qw[3], qw[4], qw[5], qw[6], qw[7]};
        asm volatile("" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]));
        asm volatile("" : "+v"(w[4]), "+v"(w[5]), "+v"(w[6]), "+v"(w[7]));
        float f[16];
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            f[e] = bf16_to_f32((w[e >> 1] >> (16 * (e & 1))) & 0xffffu) * scale[qd0 + e];
            amax = fmaxf(amax, fabsf(f[e]));
        }
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));   // the head's 32 lanes
        float alpha = amax * (float)(1.0 / 127.0);
        alpha = alpha < 1e-12f ? 1e-12f : alpha;
        const float inv = 1.0f / alpha;
        uint32_t hiw[4] = {0, 0, 0, 0}, low[4] = {0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float x = clamp127(f[e] * inv);
            const float hi = __builtin_rintf(x);
            const float lo = __builtin_rintf((x - hi) * 127.0f);
            hiw[e >> 2] |= ((uint32_t)(int32_t)hi & 0xffu) << (8 * (e & 3));
            low[e >> 2] |= ((uint32_t)(int32_t)lo & 0xffu) << (8 * (e & 3));
        }
        int8_t *stage = s.v;
        *reinterpret_cast<v4i *>(stage + row_of(qh, 0) * D + qd0) = v4i{(int)hiw[0], (int)hiw[1], (int)hiw[2], (int)hiw[3]};
        *reinterpret_cast<v4i *>(stage + row_of(qh, 1) * D + qd0) = v4i{(int)low[0], (int)low[1], (int)low[2], (int)low[3]};
        if ((tid & 31) == 0) s.asc[qh] = alpha * p.softmaxScale;
        if (DEBUG) {
            if (dbg.qcodes) {
                int8_t *qc = reinterpret_cast<int8_t *>(dbg.qcodes) + (((int64_t)t * 2 + kind) * 16) * D;
                *reinterpret_cast<v4i *>(qc + qh * D + qd0) = v4i{(int)hiw[0], (int)hiw[1], (int)hiw[2], (int)hiw[3]};
                *reinterpret_cast<v4i *>(qc + (8 + qh) * D + qd0) = v4i{(int)low[0], (int)low[1], (int)low[2], (int)low[3]};
            }
            if (dbg.alpha && (tid & 31) == 0)
                reinterpret_cast<float *>(dbg.alpha)[((int64_t)t * 2 + kind) * 8 + qh] = alpha;
        }
        __syncthreads();
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) qa[jj] = *reinterpret_cast<const v4i *>(stage + n * D + 64 * jj + 16 * g);
        asc[0] = s.asc[2 * g];
        asc[1] = s.asc[2 * g + 1];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) sc[jj] = s.scale[kind][c0 + 16 * jj + n];
        cur_kind = kind;
        __syncthreads();
    };

    for (int first = 0; first < my_tiles; first += CODE_TILES) {
        build_codes(first);
        const int ntiles = my_tiles - first < CODE_TILES ? my_tiles - first : CODE_TILES;
        {
            const int kind0 = part + S * first >= m.t0;
            if (kind0 != cur_kind) encode_q(kind0);
            load_tile(0, kind0);
        }
        for (int i = 0; i < ntiles; ++i) {
            const int k = part + S * (first + i);
            const int kind = k < m.t0 ? 0 : 1;
            const int start = (k - (kind ? m.t0 : 0)) * N;
            const int klen = kind ? m.list_len : m.ori_count;

            // ---- QK: S[16 rows][32 keys of this wave] (reference.py:286-289) ----
            v4i sacc[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                v4i acc = {0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < 8; ++j) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[j], kq[8 * kb + j], acc, 0, 0, 0);
                sacc[kb] = acc;
            }
            // ---- the same rows become the V tile ----
            bool valid[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int key = 32 * wave + 16 * kb + n;
                valid[kb] = s.code[i * N + key] >= 0;
                int8_t *row = s.v + vrow(key) + 16 * g;
#pragma unroll
                for (int j = 0; j < 8; ++j) *reinterpret_cast<v4i *>(row + 64 * j) = kq[8 * kb + j];
            }
            // Prefetch the next tile into the same registers while softmax and
            // PV run (a kind change re-encodes Q first, at the end of the tile).
            const bool more = i + 1 < ntiles;
            const int next_kind = part + S * (first + i + 1) >= m.t0;
            if (more && next_kind == cur_kind) load_tile(i + 1, next_kind);

            // ---- logits, running max (reference.py:288-303) ----
            float lg[2][2], tmax[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const int key = 32 * wave + 16 * kb + n;
                    const int32_t hi = sacc[kb][2 * hh], lo = sacc[kb][2 * hh + 1];
                    float dots = (float)hi;
                    dots = dots + (float)lo * (float)(1.0 / 127.0);
                    float l = dots * asc[hh];
                    lg[kb][hh] = valid[kb] ? l : -1e30f;
                    if (DEBUG && dbg.scores && start + key < klen) {
                        int32_t *drow = reinterpret_cast<int32_t *>(dbg.scores) + ((int64_t)t * positions + (kind ? 128 : 0) + start + key) * 16;
                        drow[2 * g + hh] = hi;
                        drow[8 + 2 * g + hh] = lo;
                    }
                }
                tmax[hh] = row16_max(fmaxf(lg[0][hh], lg[1][hh]));
            }
            if (n == 0) {
                s.red[0][wave][2 * g] = tmax[0];
                s.red[0][wave][2 * g + 1] = tmax[1];
            }
            __syncthreads();
            float mnew[2], factor[2], wsum[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int h = 2 * g + hh;
                float mm = mx[hh];
#pragma unroll
                for (int w = 0; w < WAVES; ++w) mm = fmaxf(mm, s.red[0][w][h]);
                mnew[hh] = mm;
                factor[hh] = sk_expf(mx[hh] - mnew[hh]);
            }
            // ---- weights, pairwise tile sum, P codes (reference.py:304-312) ----
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                float part_sum[2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const int key = 32 * wave + 16 * kb + n;
                    const float w = sk_expf(lg[kb][hh] - mnew[hh]);
                    const float x = w * 127.0f;
                    const float ph = __builtin_rintf(x);
                    const float pl = __builtin_rintf((x - ph) * 127.0f);
                    s.p[row_of(2 * g + hh, 0) * PROW + key] = (int8_t)(int32_t)ph;
                    s.p[row_of(2 * g + hh, 1) * PROW + key] = (int8_t)(int32_t)pl;
                    if (DEBUG && dbg.probs && start + key < klen) {
                        int8_t *drow = reinterpret_cast<int8_t *>(dbg.probs) + ((int64_t)t * positions + (kind ? 128 : 0) + start + key) * 16;
                        drow[2 * g + hh] = (int8_t)(int32_t)ph;
                        drow[8 + 2 * g + hh] = (int8_t)(int32_t)pl;
                    }
                    part_sum[kb] = row16_tree_sum(w);
                }
                wsum[hh] = part_sum[0] + part_sum[1];   // this wave's 32 keys
            }
            if (n == 0) {
                s.red[1][wave][2 * g] = wsum[0];
                s.red[1][wave][2 * g + 1] = wsum[1];
            }
            __syncthreads();
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                // Pairwise over the four 32-key blocks.
                const int h = 2 * g + hh;
                const float tile_sum = (s.red[1][0][h] + s.red[1][1][h]) + (s.red[1][2][h] + s.red[1][3][h]);
                den[hh] = den[hh] * factor[hh] + tile_sum;
            }

            // ---- PV: [16 rows][this wave's 128 columns] (reference.py:310-316) ----
            v4i vacc[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) vacc[j] = v4i{0, 0, 0, 0};
            lds_i8 *vbase = (lds_i8 *)(s.v);   // generic -> LDS address space
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                // A: P row n, keys 64 kb + 16 g .. + 15.  B: two transposed
                // 8-key reads; lanes 2r / 2r+1 address the two 8-column halves
                // of key row r, lane n receives column n of the 16-column block.
                const v4i pa = *reinterpret_cast<const v4i *>(s.p + n * PROW + 64 * kb + 16 * g);
                const int krow = 64 * kb + 16 * g + (n >> 1);
                const int lo_addr = vrow(krow) + c0 + 8 * (n & 1);
                const int hi_addr = vrow(krow + 8) + c0 + 8 * (n & 1);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const v2i b0 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(reinterpret_cast<lds_v2i *>(vbase + lo_addr + 16 * j));
                    const v2i b1 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(reinterpret_cast<lds_v2i *>(vbase + hi_addr + 16 * j));
                    const v4i vb = {b0.x, b0.y, b1.x, b1.y};
                    vacc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vb, vacc[j], 0, 0, 0);
                }
            }
            if (DEBUG && dbg.values && k < (int)dbg.tileCapacity) {
                int32_t *vout = reinterpret_cast<int32_t *>(dbg.values) + ((int64_t)t * dbg.tileCapacity + k) * 16 * D;
#pragma unroll
                for (int j = 0; j < 8; ++j)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        vout[(2 * g + hh) * D + c0 + 16 * j + n] = vacc[j][2 * hh];
                        vout[(8 + 2 * g + hh) * D + c0 + 16 * j + n] = vacc[j][2 * hh + 1];
                    }
            }
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float dots = (float)vacc[j][2 * hh];
                    dots = dots + (float)vacc[j][2 * hh + 1] * (float)(1.0 / 127.0);
                    const float pv = dots * sc[j] * (float)(1.0 / 127.0);
                    num[hh][j] = num[hh][j] * factor[hh] + pv;
                }
                mx[hh] = mnew[hh];
            }
            __syncthreads();
            if (more && next_kind != cur_kind) {
                encode_q(next_kind);
                load_tile(i + 1, next_kind);
            }
        }
    }

    if (S == 1) {
        // ---- finalize (reference.py:317-323 with one partition) ----
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int h = 2 * g + hh;
#pragma unroll
            for (int j = 0; j < 8; ++j) out_row[h * D + c0 + 16 * j + n] = (uint16_t)f32_to_bf16(num[hh][j] / den[hh]);
            if (lse_row && wave == 0 && n == 0) lse_row[h] = mx[hh] + logf(den[hh]);
        }
        return;
    }

    // ---- publish this partition: [num 512, max, den] per head ----
    float *row_partial = reinterpret_cast<float *>(p.partial) + (int64_t)t * S * HEADS * PART_FLOATS;
    const __amdgpu_buffer_rsrc_t states = row_states(row_partial);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const int h = 2 * g + hh;
        const int base = ((part * HEADS + h) * PART_FLOATS) * 4;   // byte offset in the row's states
#pragma unroll
        for (int j = 0; j < 8; ++j)
            state_store<SC1>(num[hh][j], states, base + (c0 + 16 * j + n) * 4);
        if (wave == 0 && n == 0) {
            state_store<SC1>(mx[hh], states, base + 512 * 4);
            state_store<SC1>(den[hh], states, base + 513 * 4);
        }
    }
    if (!fused) return;

    // ---- the last partition of the row to finish folds all of them ----
    // Every state store above has completed (vmcnt 0) before the ticket is
    // taken; the partition that takes the last ticket reads the states back
    // with device-coherent (sc1) loads.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t *tickets = reinterpret_cast<uint32_t *>(p.workspace);
    if (tid == 0) s.misc[5] = (int)__hip_atomic_fetch_add(&tickets[t], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s.misc[5] != S - 1) return;
    if (tid == 0) __hip_atomic_store(&tickets[t], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    fold_row<SC1>(states, S, tid, out_row, lse_row);
}

// Partition merge as a second launch (merge mode 1): one 256-thread group
// per query row, the same fold as the attention kernel's last partition.
// Rows that partition 0 marked as graph padding keep the zeros it wrote.
__global__ void __launch_bounds__(256)
c8_merge(const SharedKVArgs p, uint32_t splits)
{
    const int t = blockIdx.x, S = (int)splits;
    float *row_partial = reinterpret_cast<float *>(p.partial) + (int64_t)t * S * HEADS * PART_FLOATS;
    uint16_t *out_row = reinterpret_cast<uint16_t *>(p.out) + (int64_t)t * HEADS * D;
    float *lse_row = p.lse ? reinterpret_cast<float *>(p.lse) + (int64_t)t * HEADS : nullptr;
    fold_row<0>(row_states(row_partial), S, threadIdx.x, out_row, lse_row);
}

// ---- INT8 cache writer (cache_write.cpp:9-88): one wave per update row ----
template <typename Index, bool Paired>
__global__ void __launch_bounds__(256)
cache_write(const CacheWriteArgs a)
{
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.tokens) return;
    const Index *slots = reinterpret_cast<const Index *>(a.slots);
    const int64_t first = (int64_t)slots[(uint64_t)row * a.slotStride];
    if (first < 0) return;
    int64_t page, offset;
    if (Paired) {
        page = first;
        offset = (int64_t)slots[(uint64_t)row * a.slotStride + a.slotColumnStride];
    } else {
        page = first / (int64_t)a.pageSize;
        offset = first % (int64_t)a.pageSize;
    }
    if (page >= (int64_t)a.pages || offset < 0 || offset >= (int64_t)a.pageSize) return;
    const uint16_t *src = reinterpret_cast<const uint16_t *>(a.updates) + (uint64_t)row * a.updateStride + lane * 8;
    const float *inv = reinterpret_cast<const float *>(a.inverseScale) + lane * 8;
    const v4i x = *reinterpret_cast<const v4i *>(src);
    const f32x4 i0 = *reinterpret_cast<const f32x4 *>(inv);
    const f32x4 i1 = *reinterpret_cast<const f32x4 *>(inv + 4);
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

int check_attention(const SharedKVArgs *a)
{
    if (!a || a->heads != HEADS || (a->ratio != 1 && a->ratio != 4 && a->ratio != 128) || a->window != WINDOW)
        return 1;
    if (a->oriBlock != BLOCK_ROWS || a->oriIndices) return 1;
    if (!a->q || !a->ori || !a->oriScale || !a->oriTable || !a->cuQ || !a->seqLens || !a->sinks || !a->out)
        return 1;
    if (a->batch == 0 || a->oriPages == 0) return 1;
    if (a->ratio != 1) {
        if (a->cmpBlock != BLOCK_ROWS || !a->cmp || !a->cmpScale || !a->cmpTable) return 1;
        if (a->cmpStride % 16 || a->cmpStride < BLOCK_ROWS * D || ((a->cmp | a->cmpScale) & 15)) return 1;
    }
    if (a->ratio == 4 && (!a->indices || a->topk == 0 || a->topk > MAX_LIST)) return 1;
    if (a->splits == 0 || a->splits > MAX_SPLITS) return 1;
    if (a->splits > 1 && (!a->partial || !a->workspace)) return 1;
    if (a->oriStride % 16 || a->oriStride < BLOCK_ROWS * D) return 1;
    if ((a->q | a->ori | a->out | a->oriScale) & 15) return 1;
    return 0;
}

int g_merge_mode = 0;   // 0: fused (last partition folds), 1: separate merge launch

template <bool DEBUG>
int launch_attention(hipStream_t stream, const SharedKVArgs *a, const SharedKVDebug *debug)
{
    if (check_attention(a)) return (int)hipErrorInvalidValue;
    if (a->tokens == 0) return (int)hipSuccess;
    const SharedKVDebug dbg = debug ? *debug : SharedKVDebug{0, 0, 0, 0, 0, 0, 0};
    const uint32_t splits = a->splits;
    const uint32_t items = a->tokens * splits;
    const uint32_t grid = (items + 7u) & ~7u;
    const uint32_t fused = splits > 1 && g_merge_mode == 0;
    if (a->ratio == 4)
        hipLaunchKernelGGL((c8_attention<4, DEBUG>), dim3(grid), dim3(THREADS), 0, stream, *a, dbg, splits, items, fused);
    else if (a->ratio == 128)
        hipLaunchKernelGGL((c8_attention<128, DEBUG>), dim3(grid), dim3(THREADS), 0, stream, *a, dbg, splits, items, fused);
    else
        hipLaunchKernelGGL((c8_attention<1, DEBUG>), dim3(grid), dim3(THREADS), 0, stream, *a, dbg, splits, items, fused);
    if (splits > 1 && !fused)
        hipLaunchKernelGGL(c8_merge, dim3(a->tokens), dim3(256), 0, stream, *a, splits);
    return (int)hipGetLastError();
}

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
    return launch_sharedkv_c8_sparse(blocks, stream, args);
}

int launch_sharedkv_c8_dense(uint32_t blocks, void *stream, const SharedKVArgs *args)
{
    if (!blocks) return (int)hipSuccess;
    if (!args || (args->ratio != 128 && args->ratio != 1)) return (int)hipErrorInvalidValue;
    return launch_attention<false>(static_cast<hipStream_t>(stream), args, nullptr);
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
    if (a->tokens == 0) return (int)hipSuccess;
    const dim3 grid((a->tokens + 3) / 4);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (a->int64Slots) {
        if (a->pairedSlots) hipLaunchKernelGGL((cache_write<int64_t, true>), grid, dim3(256), 0, s, *a);
        else hipLaunchKernelGGL((cache_write<int64_t, false>), grid, dim3(256), 0, s, *a);
    } else {
        if (a->pairedSlots) hipLaunchKernelGGL((cache_write<int32_t, true>), grid, dim3(256), 0, s, *a);
        else hipLaunchKernelGGL((cache_write<int32_t, false>), grid, dim3(256), 0, s, *a);
    }
    return (int)hipGetLastError();
}

uint64_t sharedkv_c8_workspace_bytes(uint32_t tokens, uint32_t splits)
{
    (void)splits;
    return ((uint64_t)tokens * 4 + 255) / 256 * 256;
}

uint64_t sharedkv_c8_partial_bytes(uint32_t tokens, uint32_t splits)
{
    return splits > 1 ? (uint64_t)tokens * splits * HEADS * PART_FLOATS * 4 : 0;
}

int sharedkv_c8_set_merge_mode(int mode)
{
    if (mode != 0 && mode != 1) return (int)hipErrorInvalidValue;
    g_merge_mode = mode;
    return (int)hipSuccess;
}

uint32_t sharedkv_attention_args_size(void) { return (uint32_t)sizeof(SharedKVArgs); }
uint32_t sharedkv_cache_args_size(void) { return (uint32_t)sizeof(CacheWriteArgs); }
uint32_t sharedkv_abi_version(void) { return 3; }

}  // extern "C"
