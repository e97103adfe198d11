// Uniform grid over the sites and exact nearest-site queries, gfx950: the start-cell locator of the traversals.
//
// The reference locates start cells on the host with scipy's cKDTree (sites.py:38-39, called per camera centre
// in bench_infer.py:60 and eval_scene.py:69, and per ray origin for ray batches). Here the sites are binned into a
// uniform grid by a counting sort on the GPU (histogram, exclusive scan, scatter), and each query scans Chebyshev
// rings of grid cells around its own cell until no unscanned cell can hold a closer site. Distances are computed in
// float64, as cKDTree computes them, and ties go to the smaller site index, so the answer is cKDTree's except
// where two sites are at exactly the same float64 distance.
#include <mutex>

#include "vgr_abi.h"
#include "vgr_device.h"
#include "vgr_scan.h"

namespace vgr {
namespace {

constexpr int kBlock = 256;
constexpr int64_t kMaxCells = int64_t(kScanTile) * kScanTile;

struct Geom {
    float lo[3];    // grid origin
    float cell[3];  // cell edge per axis
    int res[3];     // cells per axis
};

__device__ __forceinline__ int axis_cell(float x, float lo, float cell, int res) {
    const int c = static_cast<int>(floorf((x - lo) / cell));
    return min(max(c, 0), res - 1);
}

__device__ __forceinline__ const float* site_ptr(const float* pts, int stride, int64_t i) { return pts + stride * i; }

// Cell of every site, and the number of sites per cell.
__global__ void __launch_bounds__(kBlock) grid_count(const float* __restrict__ pts, int stride, int64_t n, Geom g,
                                                     int* __restrict__ cell_of, int* __restrict__ count) {
    const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    const float* p = site_ptr(pts, stride, i);
    const int cx = axis_cell(p[0], g.lo[0], g.cell[0], g.res[0]);
    const int cy = axis_cell(p[1], g.lo[1], g.cell[1], g.res[1]);
    const int cz = axis_cell(p[2], g.lo[2], g.cell[2], g.res[2]);
    const int c = (cz * g.res[1] + cy) * g.res[0] + cx;
    cell_of[i] = c;
    atomicAdd(count + c, 1);
}

// Scatter: every site takes the next slot of its cell (the order within a cell is arbitrary; queries do not
// depend on it).
__global__ void __launch_bounds__(kBlock) grid_fill(int64_t n, const int* __restrict__ cell_of,
                                                    int* __restrict__ cursor, int* __restrict__ cell_sites) {
    const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    cell_sites[atomicAdd(cursor + cell_of[i], 1)] = static_cast<int>(i);
}

// The build's cell-ordered copy of the sites: slot s of cell_sites gets (x, y, z, bits of the site index).
__global__ void __launch_bounds__(kBlock) grid_cell_points(const float* __restrict__ pts, int stride, int64_t n,
                                                           const int* __restrict__ cell_sites, float4* __restrict__ cp) {
    const int64_t s = int64_t(blockIdx.x) * kBlock + threadIdx.x;
    if (s >= n) return;
    const int k = cell_sites[s];
    const float* p = site_ptr(pts, stride, k);
    cp[s] = make_float4(p[0], p[1], p[2], __int_as_float(k));
}

// Fills n ints with zero (the counters of a build; a kernel rather than hipMemsetAsync, so that a build is made of
// kernel launches only).
__global__ void __launch_bounds__(kBlock) zero_ints(int* __restrict__ a, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
    if (i < n) a[i] = 0;
}

// Scratch of vgr_grid_build_noalloc: 2^24 ints (64 MiB), enough for vgr_grid_work_size of 8M sites over 4M cells
// (the largest benchmark scene at two sites per cell is 12M ints). Each GPU that runs the library holds its own copy
// until the process ends. Host code never passes `scratch` itself to a kernel (in host code the name is only a
// stand-in for the symbol); it uses the device address from hipGetSymbolAddress, one per device.
constexpr int64_t kScratchInts = VGR_GRID_NOALLOC_MAX_WORK;
static __device__ __align__(256) int scratch[kScratchInts];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
int* g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch`, looked up on the first call on each device (with that device current).
int scratch_on_current_device(int** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return launch_status("grid_build_noalloc: hipGetDevice");
    VGR_REQUIRE(dev >= 0 && dev < kMaxDevices, "grid_build_noalloc: device %d beyond the %d supported", dev,
                kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess)
            return fail(VGR_ERR_LAUNCH, "grid_build_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(err));
        g_scratch_ptr[dev] = static_cast<int*>(p);
    }
    *out = g_scratch_ptr[dev];
    return VGR_OK;
}

// Nearest site of each query: lexicographic argmin of (float64 squared distance, site index).
//
// Rings r = 0, 1, ... of cells at Chebyshev distance r from the query's (clamped) cell are scanned. Every unscanned
// site lies in the grid box beyond a face of the scanned block that is not on the grid boundary, so after ring r
// no unscanned site is closer than the distance lb from the query to the nearest such region (for a query outside
// the grid, that includes its distance to the grid); the scan stops once the best distance is below lb (shrunk by
// a margin covering the float32 rounding of cell assignment), or when the block covers the grid.
// CP: the sites' positions come from the build's cell-ordered copy (grid_cell_points: the sites of a cell, and of a
// row of cells, share lines) instead of through the site index into the point array (a line per site).
template <bool CP>
__global__ void __launch_bounds__(kBlock) grid_nearest(const float* __restrict__ pts, int stride, Geom g,
                                                       const int* __restrict__ cell_start,
                                                       const int* __restrict__ cell_sites,
                                                       const float4* __restrict__ cp, const float* __restrict__ q,
                                                       int64_t m, const int* __restrict__ order, double margin,
                                                       int* __restrict__ out) {
    const int64_t t = int64_t(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= m) return;
    const int64_t i = order != nullptr ? order[t] : t;  // the query this lane answers (a permutation entry)
    if (i < 0 || i >= m) return;
    const double qx = q[3 * i], qy = q[3 * i + 1], qz = q[3 * i + 2];
    const int c[3] = {axis_cell(static_cast<float>(qx), g.lo[0], g.cell[0], g.res[0]),
                      axis_cell(static_cast<float>(qy), g.lo[1], g.cell[1], g.res[1]),
                      axis_cell(static_cast<float>(qz), g.lo[2], g.cell[2], g.res[2])};
    const double qa[3] = {qx, qy, qz};
    double best = 1e300;
    int best_k = INT_MAX;
    const auto visit = [&](int x, int y, int z) {
        const int cell = (z * g.res[1] + y) * g.res[0] + x;
        for (int s = cell_start[cell], e = cell_start[cell + 1]; s < e; ++s) {
            float px, py, pz;
            int k;
            if constexpr (CP) {
                const float4 v = cp[s];
                px = v.x, py = v.y, pz = v.z, k = __float_as_int(v.w);
            } else {
                k = cell_sites[s];
                const float* p = site_ptr(pts, stride, k);
                px = p[0], py = p[1], pz = p[2];
            }
            const double dx = qx - px, dy = qy - py, dz = qz - pz;
            const double d2 = dx * dx + dy * dy + dz * dz;
            if (d2 < best || (d2 == best && k < best_k)) best = d2, best_k = k;
        }
    };
    const int r_max = max(max(g.res[0], g.res[1]), g.res[2]);
    for (int r = 0; r <= r_max; ++r) {
        // the cells at Chebyshev distance exactly r, clipped to the grid: whole rows where z or y is on the shell,
        // the two end cells of the other rows
        const int z0 = max(c[2] - r, 0), z1 = min(c[2] + r, g.res[2] - 1);
        const int y0 = max(c[1] - r, 0), y1 = min(c[1] + r, g.res[1] - 1);
        const int x0 = max(c[0] - r, 0), x1 = min(c[0] + r, g.res[0] - 1);
        for (int z = z0; z <= z1; ++z) {
            for (int y = y0; y <= y1; ++y) {
                if (z == c[2] - r || z == c[2] + r || y == c[1] - r || y == c[1] + r) {
                    for (int x = x0; x <= x1; ++x) visit(x, y, z);
                } else {
                    if (c[0] - r >= 0) visit(c[0] - r, y, z);
                    if (r > 0 && c[0] + r < g.res[0]) visit(c[0] + r, y, z);
                }
            }
        }
        // unscanned sites lie in the grid box beyond an open face of the scanned block: the squared distance from
        // the query to each such region (an axis-aligned box) bounds theirs
        double lb2 = 1e300;
        bool open = false;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
#pragma unroll
            for (int side = 0; side < 2; ++side) {
                if (side == 0 ? c[a] - r <= 0 : c[a] + r >= g.res[a] - 1) continue;  // on the grid boundary
                open = true;
                double d2 = 0.0;
#pragma unroll
                for (int b = 0; b < 3; ++b) {
                    double lo = g.lo[b], hi = double(g.lo[b]) + double(g.res[b]) * g.cell[b];
                    if (b == a) {
                        if (side == 0) hi = double(g.lo[a]) + double(c[a] - r) * g.cell[a];
                        else lo = double(g.lo[a]) + double(c[a] + r + 1) * g.cell[a];
                    }
                    const double gap = fmax(fmax(lo - qa[b], qa[b] - hi), 0.0);
                    d2 += gap * gap;
                }
                lb2 = fmin(lb2, d2);
            }
        }
        if (!open) break;  // the scanned block covers the grid
        const double lb = sqrt(lb2) - margin;
        if (lb > 0.0 && best < lb * lb) break;
    }
    out[i] = best_k;
}

// float32 cell assignment can put a site one rounding step across a cell face: the stopping bound shrinks by a few
// float32 ulps of the grid's extent.
double nearest_margin(const float* lo, const float* cell, const int32_t* res) {
    double extent = 0.0;
    for (int a = 0; a < 3; ++a)
        extent = fmax(extent, fabs(double(lo[a])) + double(cell[a]) * res[a]);
    return extent * 1e-6;
}

Geom make_geom(const float* lo, const float* cell, const int32_t* res) {
    Geom g{};
    for (int a = 0; a < 3; ++a) g.lo[a] = lo[a], g.cell[a] = cell[a], g.res[a] = res[a];
    return g;
}

int check_geom(const float* lo, const float* cell, const int32_t* res, int64_t* n_cells) {
    VGR_REQUIRE(lo && cell && res, "grid: null geometry pointer");
    int64_t g = 1;
    for (int a = 0; a < 3; ++a) {
        VGR_REQUIRE(res[a] >= 1 && res[a] <= 65536, "grid: res[%d] must be in [1, 65536] (got %d)", a, res[a]);
        VGR_REQUIRE(cell[a] > 0.f, "grid: cell edge %d must be > 0", a);
        g *= res[a];
    }
    VGR_REQUIRE(g <= kMaxCells, "grid: at most %lld cells (got %lld)", static_cast<long long>(kMaxCells),
                static_cast<long long>(g));
    *n_cells = g;
    return VGR_OK;
}

}  // namespace
}  // namespace vgr

extern "C" int64_t vgr_grid_work_size(int64_t n_sites, int64_t n_cells) {
    const int64_t tiles = (n_cells + vgr::kScanTile - 1) / vgr::kScanTile;
    return n_sites + n_cells + tiles + 1;
}

namespace vgr {
namespace {

// Counting sort of the sites into the grid's cells, with `work` (vgr_grid_work_size ints) for the cell of every
// site, the per-cell counters (then fill cursors) and the scan's tile sums. zero_by_kernel: clear the counters with
// a kernel (the no-alloc entry point) rather than hipMemsetAsync.
int grid_build(const float* points, int64_t n_sites, int32_t stride, const float* lo, const float* cell,
               const int32_t* res, int32_t* cell_start, int32_t* cell_sites, int32_t* work, bool zero_by_kernel,
               void* stream) {
    int64_t n_cells = 0;
    if (int rc = check_geom(lo, cell, res, &n_cells)) return rc;
    VGR_REQUIRE(n_sites >= 0 && n_sites <= INT_MAX, "grid_build: n_sites must be in [0, 2^31) (got %lld)",
                static_cast<long long>(n_sites));
    VGR_REQUIRE(stride >= 3, "grid_build: stride must be >= 3 floats (got %d)", stride);
    VGR_REQUIRE(cell_start && work && (n_sites == 0 || (points && cell_sites)), "grid_build: null pointer");
    const hipStream_t s = as_stream(stream);
    const Geom g = make_geom(lo, cell, res);
    int* cell_of = work;
    int* count = work + n_sites;
    int* tile_sum = count + n_cells;
    if (zero_by_kernel) {
        hipLaunchKernelGGL(zero_ints, dim3(grid_for(n_cells, kBlock)), dim3(kBlock), 0, s, count, n_cells);
        if (int rc = launch_status("grid_build zero_ints")) return rc;
    } else if (hipMemsetAsync(count, 0, sizeof(int) * n_cells, s) != hipSuccess) {
        return launch_status("grid_build memset");
    }
    if (n_sites > 0) {
        hipLaunchKernelGGL(grid_count, dim3(grid_for(n_sites, kBlock)), dim3(kBlock), 0, s, points, int(stride),
                           n_sites, g, cell_of, count);
        if (int rc = launch_status("grid_count")) return rc;
    }
    exclusive_scan(count, n_cells, cell_start, count, tile_sum, s);  // count becomes the fill cursor
    if (int rc = launch_status("grid_build scan")) return rc;
    if (n_sites > 0) {
        hipLaunchKernelGGL(grid_fill, dim3(grid_for(n_sites, kBlock)), dim3(kBlock), 0, s, n_sites, cell_of, count,
                           cell_sites);
        return launch_status("grid_fill");
    }
    return VGR_OK;
}

}  // namespace
}  // namespace vgr

extern "C" int vgr_grid_build(const float* points, int64_t n_sites, int32_t stride, const float* lo, const float* cell,
                              const int32_t* res, int32_t* cell_start, int32_t* cell_sites, int32_t* work,
                              void* stream) {
    return vgr::grid_build(points, n_sites, stride, lo, cell, res, cell_start, cell_sites, work, false, stream);
}

extern "C" int vgr_grid_build_noalloc(const float* points, int64_t n_sites, int32_t stride, const float* lo,
                                      const float* cell, const int32_t* res, int32_t* cell_start,
                                      int32_t* cell_sites, void* stream) {
    using namespace vgr;
    int64_t n_cells = 0;
    if (int rc = check_geom(lo, cell, res, &n_cells)) return rc;
    VGR_REQUIRE(n_sites >= 0 && n_sites <= INT_MAX, "grid_build_noalloc: n_sites must be in [0, 2^31) (got %lld)",
                static_cast<long long>(n_sites));
    const int64_t need = vgr_grid_work_size(n_sites, n_cells);
    VGR_REQUIRE(need <= kScratchInts,
                "grid_build_noalloc: %lld sites over %lld cells need %lld scratch ints, beyond the static %lld; use "
                "vgr_grid_build with a workspace",
                static_cast<long long>(n_sites), static_cast<long long>(n_cells), static_cast<long long>(need),
                static_cast<long long>(kScratchInts));
    int* work = nullptr;
    if (int rc = scratch_on_current_device(&work)) return rc;
    return grid_build(points, n_sites, stride, lo, cell, res, cell_start, cell_sites, work, true, stream);
}

extern "C" int vgr_grid_nearest(const float* points, int64_t n_sites, int32_t stride, const float* lo,
                                const float* cell, const int32_t* res, const int32_t* cell_start,
                                const int32_t* cell_sites, const float* queries, int64_t n_queries, int32_t* site,
                                void* stream) {
    using namespace vgr;
    int64_t n_cells = 0;
    if (int rc = check_geom(lo, cell, res, &n_cells)) return rc;
    VGR_REQUIRE(n_queries >= 0, "grid_nearest: n_queries must be >= 0");
    if (n_queries == 0) return VGR_OK;
    VGR_REQUIRE(n_sites >= 1 && n_sites <= INT_MAX, "grid_nearest: n_sites must be in [1, 2^31) (got %lld)",
                static_cast<long long>(n_sites));
    VGR_REQUIRE(stride >= 3, "grid_nearest: stride must be >= 3 floats (got %d)", stride);
    VGR_REQUIRE(points && cell_start && cell_sites && queries && site, "grid_nearest: null pointer");
    const Geom g = make_geom(lo, cell, res);
    hipLaunchKernelGGL(grid_nearest<false>, dim3(grid_for(n_queries, kBlock)), dim3(kBlock), 0, as_stream(stream),
                       points, int(stride), g, cell_start, cell_sites, nullptr, queries, n_queries, nullptr,
                       nearest_margin(lo, cell, res), site);
    return launch_status("grid_nearest");
}

extern "C" int vgr_grid_cell_points(const float* points, int64_t n_sites, int32_t stride, const int32_t* cell_sites,
                                    float* cell_points, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(n_sites >= 0 && n_sites <= INT_MAX, "grid_cell_points: n_sites must be in [0, 2^31) (got %lld)",
                static_cast<long long>(n_sites));
    VGR_REQUIRE(stride >= 3, "grid_cell_points: stride must be >= 3 floats (got %d)", stride);
    if (n_sites == 0) return VGR_OK;
    VGR_REQUIRE(points && cell_sites && cell_points, "grid_cell_points: null pointer");
    VGR_REQUIRE(reinterpret_cast<uintptr_t>(cell_points) % 16 == 0, "grid_cell_points: cell_points must be 16-byte "
                "aligned");
    hipLaunchKernelGGL(grid_cell_points, dim3(grid_for(n_sites, kBlock)), dim3(kBlock), 0, as_stream(stream), points,
                       int(stride), n_sites, cell_sites, reinterpret_cast<float4*>(cell_points));
    return launch_status("grid_cell_points");
}

extern "C" int vgr_grid_nearest_points(const float* cell_points, int64_t n_sites, const float* lo, const float* cell,
                                       const int32_t* res, const int32_t* cell_start, const float* queries,
                                       int64_t n_queries, const int32_t* order, int32_t* site, void* stream) {
    using namespace vgr;
    int64_t n_cells = 0;
    if (int rc = check_geom(lo, cell, res, &n_cells)) return rc;
    VGR_REQUIRE(n_queries >= 0, "grid_nearest_points: n_queries must be >= 0");
    if (n_queries == 0) return VGR_OK;
    VGR_REQUIRE(n_sites >= 1 && n_sites <= INT_MAX, "grid_nearest_points: n_sites must be in [1, 2^31) (got %lld)",
                static_cast<long long>(n_sites));
    VGR_REQUIRE(cell_points && cell_start && queries && site, "grid_nearest_points: null pointer");
    VGR_REQUIRE(reinterpret_cast<uintptr_t>(cell_points) % 16 == 0, "grid_nearest_points: cell_points must be "
                "16-byte aligned");
    const Geom g = make_geom(lo, cell, res);
    hipLaunchKernelGGL(grid_nearest<true>, dim3(grid_for(n_queries, kBlock)), dim3(kBlock), 0, as_stream(stream),
                       nullptr, 3, g, cell_start, nullptr, reinterpret_cast<const float4*>(cell_points), queries,
                       n_queries, order, nearest_margin(lo, cell, res), site);
    return launch_status("grid_nearest (cell points)");
}
