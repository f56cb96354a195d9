// Data-movement floor of an attention launch (measurement kernel for
// bench.py; not part of the attention library's C ABI).
//
// One work-group of 8 waves per work item, the same grid and the same
// XCD-aware item order as the attention kernel (c8_attention), each item
// copying its tiles of 128 rows x 512 bytes from HBM into a two-tile LDS
// ring with the same LDS DMA instruction (global_load_lds_dwordx4, 16 bytes
// per lane, non-temporal when asked), eight instructions per wave and tile,
// two tiles in flight.  The row addresses of every item come precomputed in
// one flat array, so the launch has one metadata round trip (the address
// load) and no compute, no barriers and no merge: it measures how fast the
// memory system delivers exactly the rows an attention launch gathers, at
// the launch's concurrency.  Given contiguous addresses it measures a
// streaming read of the same byte count with the same instructions.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int THREADS = 512;
constexpr int WAVES = THREADS / 64;
constexpr int ROWS = 128;                 // rows per tile
constexpr int ROW_BYTES = 512;
constexpr int MAX_TILES = 16;             // tiles per work item
constexpr int DMA_PER_TILE = ROWS * ROW_BYTES / 1024 / WAVES;
static_assert(DMA_PER_TILE == 8, "eight 1 KiB copies per wave and tile");

struct alignas(16) FloorShared {
    uint64_t addr[MAX_TILES * ROWS];      // the item's row addresses
    int8_t ring[2][ROWS * ROW_BYTES];     // two tiles
};

// LDS DMA of 16 bytes per lane (lane l's bytes land at lds + 16 l); M0
// carries the LDS address.
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

// Copy instruction r of wave w moves the rows of keys 16 w + r (lanes 0-31)
// and 16 w + 8 + r (lanes 32-63), 32 lanes x 16 bytes each.
template <bool NT>
__device__ __forceinline__ void issue_tile(const FloorShared &s, int tile, int buf, int wave, int lane)
{
    typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
    const int h = lane >> 5, c = lane & 31;
    // The eight addresses are read before the first copy is issued (each
    // copy is a compiler barrier for LDS accesses).
    const u64x2 *rows = reinterpret_cast<const u64x2 *>(s.addr + tile * ROWS + 16 * wave + 8 * h);
    u64x2 ra[DMA_PER_TILE / 2];
#pragma unroll
    for (int r = 0; r < DMA_PER_TILE / 2; ++r) ra[r] = rows[r];
    const uint32_t dst = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const int8_t *)(s.ring[buf]) +
                         16 * wave * ROW_BYTES;
#pragma unroll
    for (int r = 0; r < DMA_PER_TILE; ++r)
        dma16<NT>(ra[r >> 1][r & 1] + (uint32_t)(c << 4),
                  (uint32_t)__builtin_amdgcn_readfirstlane((int)(dst + 2 * r * ROW_BYTES)));
}

template <bool NT>
__global__ void __launch_bounds__(THREADS, 1)
gather_floor(const uint64_t *addrs, const int32_t *tiles, uint32_t items, uint32_t grid, uint32_t max_tiles)
{
    __shared__ FloorShared s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t item = (blockIdx.x & 7u) * (grid >> 3) + (blockIdx.x >> 3);
    if (item >= items) return;
    const int nt = min(max(tiles[item], 0), (int)max_tiles);
    const uint64_t *mine = addrs + (uint64_t)item * max_tiles * ROWS;
    // Every address load is issued before any is stored: one round trip.
    constexpr int PER = MAX_TILES * ROWS / THREADS;
    uint64_t v[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int i = tid + e * THREADS;
        v[e] = i < nt * ROWS ? mine[i] : 0;
    }
#pragma unroll
    for (int e = 0; e < PER; ++e)
        if (tid + e * THREADS < nt * ROWS) s.addr[tid + e * THREADS] = v[e];
    __syncthreads();
    if (nt > 0) issue_tile<NT>(s, 0, 0, wave, lane);
    if (nt > 1) issue_tile<NT>(s, 1, 1, wave, lane);
    for (int i = 0; i < nt; ++i) {
        // Tile i has landed (this wave's copies; in issue order) once at most
        // the next tile's copies are outstanding.
        if (i + 1 < nt) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (i + 2 < nt) issue_tile<NT>(s, i + 2, i & 1, wave, lane);
    }
}

}  // namespace

extern "C" {

// addrs: INT64 [items][max_tiles][128] HBM row addresses (entries past an
// item's tile count are not read); tiles: INT32 [items], each 0..max_tiles.
// grid = items rounded up to a multiple of 8.  Returns a hipError_t.
int sharedkv_floor_gather(void *stream, const uint64_t *addrs, const int32_t *tiles, uint32_t items,
                          uint32_t max_tiles, int non_temporal)
{
    if (!addrs || !tiles || !items || !max_tiles || max_tiles > (uint32_t)MAX_TILES) return (int)hipErrorInvalidValue;
    const uint32_t grid = (items + 7u) & ~7u;
    hipLaunchKernelGGL(non_temporal ? &gather_floor<true> : &gather_floor<false>, dim3(grid), dim3(THREADS), 0,
                       static_cast<hipStream_t>(stream), addrs, tiles, items, grid, max_tiles);
    return (int)hipGetLastError();
}

}  // extern "C"
