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
// Design (one GPU, HBM bound): one work-group of 4 waves per (query row,
// KV partition).  A tile of 128 gathered 512-byte KV rows is staged in LDS
// with 16-byte loads; the same bytes serve as K (QK) and V (PV).  QK and PV
// are int8 x int8 -> int32 on v_mfma_i32_16x16x64_i8 with M = 16 rows =
// 8 heads x {code, residual}; softmax is FP32 in registers with 16-lane
// shuffles.  Integer partials are exact, so any assignment of keys to waves
// gives the reference's integers; the FP32 sequence below is kept in the
// reference's order with contraction disabled.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sharedkv_hip.h"

#pragma clang fp contract(off)

namespace {

constexpr int D = 512;
constexpr int HEADS = 8;
constexpr int N = SHAREDKV_C8_TILE;    // keys per tile
constexpr int THREADS = 256;           // 4 waves
constexpr int RS = D + 16;             // LDS row stride of a staged KV row (bytes)
constexpr int MAX_LIST = 1024;         // C4 top-k capacity of the index list
constexpr int PART_FLOATS = 520;       // per (row, split, head): 512 numerator, max, denominator
constexpr int WINDOW = 128;
constexpr int BLOCK_ROWS = 32;
constexpr uint32_t MAX_SPLITS = 16;
static_assert(N == 128, "wave/key mapping below assumes 128-key tiles");

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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
// scaled by 2^n.  The CPU oracle evaluates the identical sequence, so the
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

// 4x4 byte transpose: out[j].byte[i] = in[i].byte[j].
__device__ __forceinline__ void transpose4x4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t *c)
{
    const uint32_t e01 = __builtin_amdgcn_perm(a1, a0, 0x06020400u);
    const uint32_t o01 = __builtin_amdgcn_perm(a1, a0, 0x07030501u);
    const uint32_t e23 = __builtin_amdgcn_perm(a3, a2, 0x06020400u);
    const uint32_t o23 = __builtin_amdgcn_perm(a3, a2, 0x07030501u);
    c[0] = __builtin_amdgcn_perm(e23, e01, 0x05040100u);
    c[1] = __builtin_amdgcn_perm(o23, o01, 0x05040100u);
    c[2] = __builtin_amdgcn_perm(e23, e01, 0x07060302u);
    c[3] = __builtin_amdgcn_perm(o23, o01, 0x07060302u);
}

struct Shared {
    int8_t tile[N * RS];        // staged KV tile; Q staging [16][512] at kind switches
    int8_t prob[16 * N];        // P codes, MFMA row order
    int32_t list[MAX_LIST];     // C4 compressed index list (compacted or raw)
    uint64_t addr[2][N];        // row addresses of the current / next tile (0 = masked)
    float red[2][4][HEADS];     // per-wave max / sum exchange
    float asc[HEADS];           // alpha * softmax_scale of the current kind
    int32_t scan[4];
    int32_t misc[4];
};

// MFMA row m of the 16-row operands: rows 4g..4g+3 hold heads 2g and 2g+1,
// each as {code, residual}.  The output lane group g then owns both rows of
// both of its heads.
__device__ __forceinline__ int row_of(int head, int residual) { return 4 * (head >> 1) + 2 * (head & 1) + residual; }

struct Meta {
    int32_t batch, position, first_ori, ori_count, count, list_len, t0, total;
};

template <int RATIO, bool DEBUG>
__global__ void __launch_bounds__(THREADS, 2)
c8_attention(const SharedKVArgs p, const SharedKVDebug dbg, uint32_t splits, uint32_t items, uint32_t fused)
{
    __shared__ Shared s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, n = lane & 15;

    // XCD-aware order: consecutive work items (the partitions of one query,
    // then the next query) stay on one XCD and share its L2.
    const uint32_t G = gridDim.x;
    const uint32_t item = (blockIdx.x & 7u) * (G >> 3) + (blockIdx.x >> 3);
    if (item >= items) return;
    const int32_t t = (int32_t)(item / splits);
    const int32_t part = (int32_t)(item % splits);
    const int32_t S = (int32_t)splits;

    const int32_t *cu = reinterpret_cast<const int32_t *>(p.cuQ);
    const int32_t *lens = reinterpret_cast<const int32_t *>(p.seqLens);

    // ---- live shape (attention_impl.h:121-137) and the row's request ----
    if (tid == 0) { s.misc[0] = 0; s.misc[1] = -1; }
    __syncthreads();
    for (int b = tid + 1; b <= (int)p.batch; b += THREADS)
        if (lens[b - 1] > 0 && cu[b] >= 0) atomicMax(&s.misc[0], b);
    __syncthreads();
    const int live_batch = s.misc[0];
    const int end = live_batch ? cu[live_batch] : 0;
    const int live_tokens = end <= 0 ? 0 : (end < (int)p.tokens ? end : (int)p.tokens);
    if (t < live_tokens)
        for (int b = tid; b < live_batch; b += THREADS)
            if (cu[b] <= t && t < cu[b + 1]) s.misc[1] = b;
    __syncthreads();
    const int batch = s.misc[1];
    uint16_t *out_row = reinterpret_cast<uint16_t *>(p.out) + (int64_t)t * HEADS * D;
    float *lse_row = p.lse ? reinterpret_cast<float *>(p.lse) + (int64_t)t * HEADS : nullptr;
    if (t >= live_tokens || batch < 0) {
        // Graph padding rows are zero-filled (attention_impl.h:443-460).
        if (part == 0) {
            reinterpret_cast<v4i *>(out_row)[tid * 2] = v4i{0, 0, 0, 0};
            reinterpret_cast<v4i *>(out_row)[tid * 2 + 1] = v4i{0, 0, 0, 0};
            if (lse_row && tid < HEADS) lse_row[tid] = 0.0f;
        }
        return;
    }

    // ---- selection (attention_impl.h:58-73, reference.py:228-253) ----
    Meta m;
    m.batch = batch;
    m.position = lens[batch] - cu[batch + 1] + t;
    m.first_ori = m.position + 1 > WINDOW ? m.position + 1 - WINDOW : 0;
    m.ori_count = m.position + 1 - m.first_ori;
    if (m.ori_count < 0) m.ori_count = 0;
    m.count = (m.position + 1) / RATIO;
    if (RATIO == 4) {
        const int topk = (int)p.topk;
        const int32_t *ix = reinterpret_cast<const int32_t *>(p.indices) + (int64_t)t * topk;
        const bool compact = m.count < topk && topk <= MAX_LIST;   // reference.py:250
        int v[4], ok[4], mine = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = tid * 4 + i;
            v[i] = j < topk ? ix[j] : -1;
            ok[i] = v[i] >= 0 && v[i] < m.count;
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
            int base = 0;
            for (int w = 0; w < wave; ++w) base += s.scan[w];
            int at = base + incl - mine;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (ok[i]) s.list[at++] = v[i];
            m.list_len = s.scan[0] + s.scan[1] + s.scan[2] + s.scan[3];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = tid * 4 + i;
                if (j < topk) s.list[j] = ok[i] ? v[i] : -1;
            }
            m.list_len = topk;
        }
        __syncthreads();
    } else if (RATIO == 128) {
        m.list_len = m.count > 0 ? m.count : 0;
    } else {
        m.list_len = 0;   // window only
    }
    m.t0 = (m.ori_count + N - 1) / N;
    m.total = m.t0 + (m.list_len + N - 1) / N;

    // ---- per-lane softmax state for heads 2g and 2g+1 ----
    const float *sinks = reinterpret_cast<const float *>(p.sinks);
    float mx[2], den[2], num[2][8];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        mx[hh] = sinks[2 * g + hh];
        den[hh] = part == 0 ? 1.0f : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) num[hh][j] = 0.0f;
    }

    const int positions = 128 + (int)dbg.cmpCapacity;
    const int col0 = 128 * wave + 8 * n;   // this lane's 8 PV output columns

    // Row addresses of tile k into s.addr[slot]; threads 0..127, one row each.
    auto tile_addresses = [&](int k, int slot) {
        if (tid < N) {
            const int kind = k < m.t0 ? 0 : 1;
            const int start = (k - (kind ? m.t0 : 0)) * N;
            const int pos = start + tid;
            uint64_t a = 0;
            // Rows whose logical page lies outside the block table, or whose
            // physical page is negative or (original cache) past the pool,
            // are treated as masked instead of being dereferenced.
            if (kind == 0) {
                if (pos < m.ori_count) {
                    const int idx = m.first_ori + pos;
                    if (idx / BLOCK_ROWS < (int)p.oriTableWidth) {
                        const int32_t page = gptr<int32_t>(p.oriTable)[(int64_t)m.batch * p.oriTableWidth + idx / BLOCK_ROWS];
                        if (page >= 0 && (uint32_t)page < p.oriPages)
                            a = p.ori + (uint64_t)page * p.oriStride + (uint64_t)(idx % BLOCK_ROWS) * D;
                    }
                }
            } else if (pos < m.list_len) {
                const int idx = RATIO == 4 ? s.list[pos] : pos;
                if (idx >= 0 && idx / BLOCK_ROWS < (int)p.cmpTableWidth) {
                    const int32_t page = gptr<int32_t>(p.cmpTable)[(int64_t)m.batch * p.cmpTableWidth + idx / BLOCK_ROWS];
                    if (page >= 0) a = p.cmp + (uint64_t)page * p.cmpStride + (uint64_t)(idx % BLOCK_ROWS) * D;
                }
            }
            s.addr[slot][tid] = a;
        }
    };
    // 16-byte chunk c = tid + 256 i of the tile: row c / 32, column (c % 32) * 16.
    auto tile_loads = [&](int slot, v4i *buf) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = (tid >> 5) + 8 * i;
            const uint64_t a = s.addr[slot][row];
            buf[i] = a ? *gptr<v4i>(a + (uint64_t)(tid & 31) * 16) : v4i{0, 0, 0, 0};
        }
    };

    v4i qa[8];            // Q codes as MFMA A operands, per 64-byte D block
    float asc[2] = {0.0f, 0.0f};
    float sc[8];          // channel scale of this lane's output columns
    int cur_kind = -1, slot = 0;
    v4i buf[16];

    int k = part;
    if (k < m.total) tile_addresses(k, 0);
    __syncthreads();
    if (k < m.total) tile_loads(0, buf);

    for (; k < m.total; k += S) {
        const int kind = k < m.t0 ? 0 : 1;
        const int start = (k - (kind ? m.t0 : 0)) * N;
        const int klen = kind ? m.list_len : m.ori_count;
        if (kind != cur_kind) {
            // ---- Q folding and residual split (reference.py:274-279) ----
            const float *scale = reinterpret_cast<const float *>(kind ? p.cmpScale : p.oriScale);
            const int h = tid >> 5, d0 = (tid & 31) * 16;
            const uint16_t *qrow = reinterpret_cast<const uint16_t *>(p.q) + ((int64_t)t * HEADS + h) * D + d0;
            const v4i q0 = *reinterpret_cast<const v4i *>(qrow);
            const v4i q1 = *reinterpret_cast<const v4i *>(qrow + 8);
            const uint32_t qw[8] = {(uint32_t)q0.x, (uint32_t)q0.y, (uint32_t)q0.z, (uint32_t)q0.w,
                                    (uint32_t)q1.x, (uint32_t)q1.y, (uint32_t)q1.z, (uint32_t)q1.w};
            float f[16];
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t bits = (qw[i >> 1] >> (16 * (i & 1))) & 0xffffu;
                f[i] = bf16_to_f32(bits) * scale[d0 + i];
                amax = fmaxf(amax, fabsf(f[i]));
            }
#pragma unroll
            for (int o = 1; o < 32; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
            float alpha = amax * (float)(1.0 / 127.0);
            alpha = alpha < 1e-12f ? 1e-12f : alpha;
            const float inv = 1.0f / alpha;
            uint32_t hiw[4] = {0, 0, 0, 0}, low[4] = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float x = clamp127(f[i] * inv);
                const float hi = __builtin_rintf(x);
                const float lo = __builtin_rintf((x - hi) * 127.0f);
                hiw[i >> 2] |= ((uint32_t)(int32_t)hi & 0xffu) << (8 * (i & 3));
                low[i >> 2] |= ((uint32_t)(int32_t)lo & 0xffu) << (8 * (i & 3));
            }
            int8_t *stage = s.tile;
            *reinterpret_cast<v4i *>(stage + row_of(h, 0) * D + d0) = v4i{(int)hiw[0], (int)hiw[1], (int)hiw[2], (int)hiw[3]};
            *reinterpret_cast<v4i *>(stage + row_of(h, 1) * D + d0) = v4i{(int)low[0], (int)low[1], (int)low[2], (int)low[3]};
            if ((tid & 31) == 0) s.asc[h] = alpha * p.softmaxScale;
            if (DEBUG) {
                if (dbg.qcodes) {
                    int8_t *qc = reinterpret_cast<int8_t *>(dbg.qcodes) + (((int64_t)t * 2 + kind) * 16) * D;
                    *reinterpret_cast<v4i *>(qc + h * D + d0) = v4i{(int)hiw[0], (int)hiw[1], (int)hiw[2], (int)hiw[3]};
                    *reinterpret_cast<v4i *>(qc + (8 + h) * D + d0) = v4i{(int)low[0], (int)low[1], (int)low[2], (int)low[3]};
                }
                if (dbg.alpha && (tid & 31) == 0)
                    reinterpret_cast<float *>(dbg.alpha)[((int64_t)t * 2 + kind) * 8 + h] = alpha;
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < 8; ++j) qa[j] = *reinterpret_cast<const v4i *>(stage + n * D + 64 * j + 16 * g);
            asc[0] = s.asc[2 * g];
            asc[1] = s.asc[2 * g + 1];
#pragma unroll
            for (int j = 0; j < 8; ++j) sc[j] = scale[col0 + j];
            cur_kind = kind;
            __syncthreads();
        }

        // ---- stage tile k; address and prefetch tile k + S ----
#pragma unroll
        for (int i = 0; i < 16; ++i)
            *reinterpret_cast<v4i *>(s.tile + ((tid >> 5) + 8 * i) * RS + (tid & 31) * 16) = buf[i];
        const int kn = k + S;
        if (kn < m.total) tile_addresses(kn, slot ^ 1);
        __syncthreads();
        if (kn < m.total) tile_loads(slot ^ 1, buf);

        // ---- QK: S[16 rows][32 keys of this wave] (reference.py:286-289) ----
        v4i sacc[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int key = 32 * wave + 16 * kb + n;
            v4i acc = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const v4i kv = *reinterpret_cast<const v4i *>(s.tile + key * RS + 64 * j + 16 * g);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[j], kv, acc, 0, 0, 0);
            }
            sacc[kb] = acc;
        }

        // ---- logits, running max (reference.py:288-303) ----
        float lg[2][2];
        float tmax[2] = {-__builtin_inff(), -__builtin_inff()};
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int key = 32 * wave + 16 * kb + n;
            const bool valid = s.addr[slot][key] != 0;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int32_t hi = sacc[kb][2 * hh], lo = sacc[kb][2 * hh + 1];
                float dots = (float)hi;
                dots = dots + (float)lo * (float)(1.0 / 127.0);
                float l = dots * asc[hh];
                l = valid ? l : -1e30f;
                lg[kb][hh] = l;
                tmax[hh] = fmaxf(tmax[hh], l);
                if (DEBUG && dbg.scores && start + key < klen) {
                    int32_t *row = reinterpret_cast<int32_t *>(dbg.scores) + ((int64_t)t * positions + (kind ? 128 : 0) + start + key) * 16;
                    row[2 * g + hh] = hi;
                    row[8 + 2 * g + hh] = lo;
                }
            }
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) tmax[hh] = fmaxf(tmax[hh], __shfl_xor(tmax[hh], o));
        if (n == 0) {
            s.red[0][wave][2 * g] = tmax[0];
            s.red[0][wave][2 * g + 1] = tmax[1];
        }
        __syncthreads();
        float mnew[2], factor[2], wsum[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int h = 2 * g + hh;
            mnew[hh] = fmaxf(fmaxf(mx[hh], fmaxf(s.red[0][0][h], s.red[0][1][h])), fmaxf(s.red[0][2][h], s.red[0][3][h]));
            factor[hh] = sk_expf(mx[hh] - mnew[hh]);
        }
        // ---- weights, pairwise tile sum, P codes (reference.py:304-312) ----
        float wk[2][2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                float w = sk_expf(lg[kb][hh] - mnew[hh]);
                wk[kb][hh] = w;
                const int key = 32 * wave + 16 * kb + n;
                const float x = w * 127.0f;
                const float ph = __builtin_rintf(x);
                const float pl = __builtin_rintf((x - ph) * 127.0f);
                s.prob[row_of(2 * g + hh, 0) * N + key] = (int8_t)(int32_t)ph;
                s.prob[row_of(2 * g + hh, 1) * N + key] = (int8_t)(int32_t)pl;
                if (DEBUG && dbg.probs && start + key < klen) {
                    int8_t *row = reinterpret_cast<int8_t *>(dbg.probs) + ((int64_t)t * positions + (kind ? 128 : 0) + start + key) * 16;
                    row[2 * g + hh] = (int8_t)(int32_t)ph;
                    row[8 + 2 * g + hh] = (int8_t)(int32_t)pl;
                }
            }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            float a = wk[0][hh], b = wk[1][hh];
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                a = a + __shfl_xor(a, o);
                b = b + __shfl_xor(b, o);
            }
            wsum[hh] = a + b;
        }
        if (n == 0) {
            s.red[1][wave][2 * g] = wsum[0];
            s.red[1][wave][2 * g + 1] = wsum[1];
        }
        __syncthreads();
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int h = 2 * g + hh;
            const float tile_sum = (s.red[1][0][h] + s.red[1][1][h]) + (s.red[1][2][h] + s.red[1][3][h]);
            den[hh] = den[hh] * factor[hh] + tile_sum;
        }

        // ---- PV: [16 rows][this wave's 128 columns] (reference.py:310-316) ----
        v4i vacc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) vacc[j] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            v4i pa;
            const int8_t *prow = s.prob + n * N + 64 * kb + 4 * g;
            pa.x = *reinterpret_cast<const int32_t *>(prow);
            pa.y = *reinterpret_cast<const int32_t *>(prow + 16);
            pa.z = *reinterpret_cast<const int32_t *>(prow + 32);
            pa.w = *reinterpret_cast<const int32_t *>(prow + 48);
            uint32_t bq[8][4];   // [column j][key quad q]
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                u32x2 r[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    r[i] = *reinterpret_cast<const u32x2 *>(s.tile + (64 * kb + 16 * q + 4 * g + i) * RS + col0);
                uint32_t lo4[4], hi4[4];
                transpose4x4(r[0].x, r[1].x, r[2].x, r[3].x, lo4);
                transpose4x4(r[0].y, r[1].y, r[2].y, r[3].y, hi4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    bq[j][q] = lo4[j];
                    bq[4 + j][q] = hi4[j];
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const v4i vb = {(int)bq[j][0], (int)bq[j][1], (int)bq[j][2], (int)bq[j][3]};
                vacc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vb, vacc[j], 0, 0, 0);
            }
        }
        if (DEBUG && dbg.values && k < (int)dbg.tileCapacity) {
            int32_t *vrow = reinterpret_cast<int32_t *>(dbg.values) + ((int64_t)t * dbg.tileCapacity + k) * 16 * D;
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    vrow[(2 * g + hh) * D + col0 + j] = vacc[j][2 * hh];
                    vrow[(8 + 2 * g + hh) * D + col0 + j] = vacc[j][2 * hh + 1];
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
        slot ^= 1;
        __syncthreads();
    }

    if (S == 1) {
        // ---- finalize (reference.py:317-323 with one partition) ----
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int h = 2 * g + hh;
            uint32_t packed[4];
#pragma unroll
            for (int j = 0; j < 8; j += 2)
                packed[j >> 1] = f32_to_bf16(num[hh][j] / den[hh]) | (f32_to_bf16(num[hh][j + 1] / den[hh]) << 16);
            *reinterpret_cast<v4i *>(out_row + h * D + col0) = v4i{(int)packed[0], (int)packed[1], (int)packed[2], (int)packed[3]};
            if (lse_row && wave == 0 && n == 0) lse_row[h] = mx[hh] + logf(den[hh]);
        }
        return;
    }

    // ---- publish this partition ----
    float *partial = reinterpret_cast<float *>(p.partial);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const int h = 2 * g + hh;
        float *dst = partial + (((int64_t)t * S + part) * HEADS + h) * PART_FLOATS;
        *reinterpret_cast<f32x4 *>(dst + col0) = f32x4{num[hh][0], num[hh][1], num[hh][2], num[hh][3]};
        *reinterpret_cast<f32x4 *>(dst + col0 + 4) = f32x4{num[hh][4], num[hh][5], num[hh][6], num[hh][7]};
        if (wave == 0 && n == 0) {
            dst[512] = mx[hh];
            dst[513] = den[hh];
        }
    }
    if (!fused) return;
    __threadfence();
    __syncthreads();
    uint32_t *tickets = reinterpret_cast<uint32_t *>(p.workspace);
    if (tid == 0) s.misc[2] = atomicAdd(&tickets[t], 1u) == (uint32_t)(S - 1);
    __syncthreads();
    if (!s.misc[2]) return;
    __threadfence();
    if (tid == 0) atomicExch(&tickets[t], 0u);

    // ---- merge the partitions (reference.py:317-323) ----
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const int h = 2 * g + hh;
        const float *src = partial + ((int64_t)t * S * HEADS + h) * PART_FLOATS;
        const int64_t step = (int64_t)HEADS * PART_FLOATS;
        float top = src[512];
        for (int sp = 1; sp < S; ++sp) top = fmaxf(top, src[sp * step + 512]);
        float acc[8], dsum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
        for (int sp = 0; sp < S; ++sp) {
            const float *ps = src + sp * step;
            const float f = sk_expf(ps[512] - top);
            const f32x4 a = *reinterpret_cast<const f32x4 *>(ps + col0);
            const f32x4 b = *reinterpret_cast<const f32x4 *>(ps + col0 + 4);
            acc[0] = acc[0] + a.x * f; acc[1] = acc[1] + a.y * f; acc[2] = acc[2] + a.z * f; acc[3] = acc[3] + a.w * f;
            acc[4] = acc[4] + b.x * f; acc[5] = acc[5] + b.y * f; acc[6] = acc[6] + b.z * f; acc[7] = acc[7] + b.w * f;
            dsum = dsum + ps[513] * f;
        }
        uint32_t packed[4];
#pragma unroll
        for (int j = 0; j < 8; j += 2)
            packed[j >> 1] = f32_to_bf16(acc[j] / dsum) | (f32_to_bf16(acc[j + 1] / dsum) << 16);
        *reinterpret_cast<v4i *>(out_row + h * D + col0) = v4i{(int)packed[0], (int)packed[1], (int)packed[2], (int)packed[3]};
        if (lse_row && wave == 0 && n == 0) lse_row[h] = top + logf(dsum);
    }
}

// Second-kernel merge (merge mode 1): one work-group per live query row.
__global__ void __launch_bounds__(THREADS)
c8_merge(const SharedKVArgs p, uint32_t splits)
{
    const int t = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, n = lane & 15;
    const int S = (int)splits;
    const int32_t *cu = reinterpret_cast<const int32_t *>(p.cuQ);
    const int32_t *lens = reinterpret_cast<const int32_t *>(p.seqLens);
    __shared__ int live;
    if (tid == 0) live = 0;
    __syncthreads();
    for (int b = tid + 1; b <= (int)p.batch; b += THREADS)
        if (lens[b - 1] > 0 && cu[b] >= 0) atomicMax(&live, b);
    __syncthreads();
    const int end = live ? cu[live] : 0;
    const int live_tokens = end <= 0 ? 0 : (end < (int)p.tokens ? end : (int)p.tokens);
    if (t >= live_tokens) return;
    int found = 0;
    for (int b = 0; b < live; ++b) found |= cu[b] <= t && t < cu[b + 1];
    if (!found) return;
    const int col0 = 128 * wave + 8 * n;
    uint16_t *out_row = reinterpret_cast<uint16_t *>(p.out) + (int64_t)t * HEADS * D;
    float *lse_row = p.lse ? reinterpret_cast<float *>(p.lse) + (int64_t)t * HEADS : nullptr;
    const float *partial = reinterpret_cast<const float *>(p.partial);
    for (int hh = 0; hh < 2; ++hh) {
        const int h = 2 * g + hh;
        const float *src = partial + ((int64_t)t * S * HEADS + h) * PART_FLOATS;
        const int64_t step = (int64_t)HEADS * PART_FLOATS;
        float top = src[512];
        for (int sp = 1; sp < S; ++sp) top = fmaxf(top, src[sp * step + 512]);
        float acc[8], dsum = 0.0f;
        for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
        for (int sp = 0; sp < S; ++sp) {
            const float *ps = src + sp * step;
            const float f = sk_expf(ps[512] - top);
            for (int j = 0; j < 8; ++j) acc[j] = acc[j] + ps[col0 + j] * f;
            dsum = dsum + ps[513] * f;
        }
        uint32_t packed[4];
        for (int j = 0; j < 8; j += 2)
            packed[j >> 1] = f32_to_bf16(acc[j] / dsum) | (f32_to_bf16(acc[j + 1] / dsum) << 16);
        *reinterpret_cast<v4i *>(out_row + h * D + col0) = v4i{(int)packed[0], (int)packed[1], (int)packed[2], (int)packed[3]};
        if (lse_row && wave == 0 && n == 0) lse_row[h] = top + logf(dsum);
    }
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

int g_merge_mode = 0;

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

template <bool DEBUG>
int launch_attention(hipStream_t stream, const SharedKVArgs *a, const SharedKVDebug *debug)
{
    if (check_attention(a)) return (int)hipErrorInvalidValue;
    if (a->tokens == 0) return (int)hipSuccess;
    const SharedKVDebug dbg = debug ? *debug : SharedKVDebug{0, 0, 0, 0, 0, 0, 0};
    const uint32_t splits = a->splits;
    const uint32_t items = a->tokens * splits;
    const uint32_t grid = (items + 7u) & ~7u;
    const uint32_t fused = g_merge_mode == 0;
    if (a->ratio == 4)
        hipLaunchKernelGGL((c8_attention<4, DEBUG>), dim3(grid), dim3(THREADS), 0, stream, *a, dbg, splits, items, fused);
    else if (a->ratio == 128)
        hipLaunchKernelGGL((c8_attention<128, DEBUG>), dim3(grid), dim3(THREADS), 0, stream, *a, dbg, splits, items, fused);
    else
        hipLaunchKernelGGL((c8_attention<1, DEBUG>), dim3(grid), dim3(THREADS), 0, stream, *a, dbg, splits, items, fused);
    if (splits > 1 && !fused)
        hipLaunchKernelGGL(c8_merge, dim3(a->tokens), dim3(THREADS), 0, stream, *a, splits);
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
uint32_t sharedkv_abi_version(void) { return 1; }

}  // extern "C"
