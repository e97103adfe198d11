// Device-wide exclusive scan of int counts for counting sorts (histogram, scan, scatter), gfx950: tiles of
// kScanTile counts are scanned by 1024-thread blocks, then the tile totals by one block (so at most kScanTile^2
// counts), then the tile offsets are added. Used by the site grid (grid.hip) and the per-site gathers of the field
// backward (field_grad.hip). Each translation unit gets its own copy of these kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vgr {
namespace {

constexpr int kScanThreads = 1024;                    // threads of a scan block
constexpr int kScanItems = 4;                         // counts per scan thread
constexpr int kScanTile = kScanThreads * kScanItems;  // counts per scan block
constexpr int kScanAddBlock = 256;

// Exclusive scan of one tile of kScanTile counts within the tile; the tile total goes to tile_sum.
__global__ void __launch_bounds__(kScanThreads) scan_tiles(const int* __restrict__ count, int64_t n_cells,
                                                           int* __restrict__ start, int* __restrict__ tile_sum) {
    __shared__ int part[kScanThreads];
    const int64_t base = int64_t(blockIdx.x) * kScanTile + int64_t(threadIdx.x) * kScanItems;
    int v[kScanItems], sum = 0;
#pragma unroll
    for (int u = 0; u < kScanItems; ++u) {
        v[u] = base + u < n_cells ? count[base + u] : 0;
        sum += v[u];
    }
    part[threadIdx.x] = sum;
    __syncthreads();
    for (int off = 1; off < kScanThreads; off <<= 1) {  // inclusive scan of the thread sums
        const int add = threadIdx.x >= off ? part[threadIdx.x - off] : 0;
        __syncthreads();
        part[threadIdx.x] += add;
        __syncthreads();
    }
    int run = part[threadIdx.x] - sum;
#pragma unroll
    for (int u = 0; u < kScanItems; ++u) {
        if (base + u < n_cells) start[base + u] = run;
        run += v[u];
    }
    if (threadIdx.x == kScanThreads - 1) tile_sum[blockIdx.x] = part[threadIdx.x];
}

// Exclusive scan of the tile totals (at most kScanTile of them) in place, by one block; the grand total goes to
// tile_sum[n_tiles].
__global__ void __launch_bounds__(kScanThreads) scan_tile_sums(int* __restrict__ tile_sum, int n_tiles) {
    __shared__ int part[kScanThreads];
    const int base = threadIdx.x * kScanItems;
    int v[kScanItems], sum = 0;
#pragma unroll
    for (int u = 0; u < kScanItems; ++u) {
        v[u] = base + u < n_tiles ? tile_sum[base + u] : 0;
        sum += v[u];
    }
    part[threadIdx.x] = sum;
    __syncthreads();
    for (int off = 1; off < kScanThreads; off <<= 1) {
        const int add = threadIdx.x >= off ? part[threadIdx.x - off] : 0;
        __syncthreads();
        part[threadIdx.x] += add;
        __syncthreads();
    }
    int run = part[threadIdx.x] - sum;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kScanItems; ++u) {
        if (base + u < n_tiles) tile_sum[base + u] = run;
        run += v[u];
    }
    if (threadIdx.x == kScanThreads - 1) tile_sum[n_tiles] = part[threadIdx.x];
}

// Adds the tile offsets: start becomes the global exclusive scan (start[n_cells] = total), and the count array is
// overwritten with it, as the fill cursor.
__global__ void __launch_bounds__(kScanAddBlock) scan_add(int* __restrict__ start, int* __restrict__ cursor, int64_t n_cells,
                                                   const int* __restrict__ tile_sum, int n_tiles) {
    const int64_t i = int64_t(blockIdx.x) * kScanAddBlock + threadIdx.x;
    if (i < n_cells) {
        const int s = start[i] + tile_sum[i / kScanTile];
        start[i] = s;
        cursor[i] = s;
    } else if (i == n_cells) {
        start[i] = tile_sum[n_tiles];
    }
}

// Bytes of int scratch the scan needs for n counts (the tile totals).
constexpr int64_t scan_tiles_of(int64_t n) { return (n + kScanTile - 1) / kScanTile; }

// start[0 .. n] = exclusive scan of count[0 .. n) (start[n] = total), cursor[0 .. n) = start[0 .. n);
// tile_sum: scan_tiles_of(n) + 1 ints. count and cursor may be the same array.
inline void exclusive_scan(const int* count, int64_t n, int* start, int* cursor, int* tile_sum, hipStream_t s) {
    const int n_tiles = static_cast<int>(scan_tiles_of(n));
    hipLaunchKernelGGL(scan_tiles, dim3(n_tiles), dim3(kScanThreads), 0, s, count, n, start, tile_sum);
    hipLaunchKernelGGL(scan_tile_sums, dim3(1), dim3(kScanThreads), 0, s, tile_sum, n_tiles);
    hipLaunchKernelGGL(scan_add, dim3(static_cast<unsigned>((n + kScanAddBlock) / kScanAddBlock)), dim3(kScanAddBlock),
                       0, s, start, cursor, n, tile_sum, n_tiles);
}

}  // namespace
}  // namespace vgr
