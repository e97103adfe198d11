// Records of the inference renderer from the model's tensors, gfx950: the step before foam_infer.
//
// Semantics follow pack_foam of the reference (render.py:179-225), with its optional Z-order renumbering
// (render.py:168-176; the permutation comes from the caller): self-first neighbourhoods (offsets of N + 1 entries,
// nbr of M + N), one float4 per edge = (p_j, half2(r2_j, lam_j)), the site records attr (N, 20) = (density conic,
// min(raw, 30), 0, colour conic, 0 x 6), the positions padded to float4, and the SH rows, all in the new numbering.
//   r2_j  = 2 max_k(s_jk^2 + floor^2) max(min(raw_j, 30) - ln eps_density, 0) (1 + 2^-9), or inf when eps_density = 0:
//           the squared distance beyond which rho_j G_j < eps_density (rounded up before the half conversion);
//   lam_j = min(1 / max_k(t_jk^2 + floor^2) (1 - 2^-9), 65000): the smallest eigenvalue of the colour conic,
//           rounded down; t the colour scales.
// Both halves are rounded to nearest even, as torch's half conversion does.
//
// Four passes, each one read of its inputs: the edge record (p, cut-off word) of every site and the inverse
// permutation, per old site; the self-first row sizes in the new numbering and their exclusive scan (the tile scan
// of vgr_scan.h); site records and SH rows per new site; edge records per new site (its row written contiguously by
// one lane, each neighbour's record gathered as one float4).
//
// vgr_morton_codes gives the Z-order keys of the renumbering, with the arithmetic of morton_order (render.py:168-176):
// q = trunc((p - lo) / max(hi - lo, 1e-12) * 1023) per axis over the bounding box [lo, hi], bit b of axis a at
// bit 3 b + a of the key; the caller sorts them.
#include "vgr_abi.h"
#include "vgr_device.h"
#include "vgr_scan.h"
#include "vgr_bbox.h"

#include <cmath>

namespace vgr {
namespace {

constexpr int kBlock = 256;

struct PackIn {
    const float* __restrict__ points;  // (N, 3)
    const int* __restrict__ offsets;   // (N + 1)
    const int* __restrict__ adj;       // (M)
    const float* __restrict__ raw;     // (N)
    const float* __restrict__ d_log_scale;  // (N, 3)
    const float* __restrict__ c_log_scale;  // (N, 3)
    const float* __restrict__ dA;      // (N, 6)
    const float* __restrict__ cA;      // (N, 6)
    const float4* __restrict__ sh;     // (N, 12) fp32
    const int* __restrict__ perm;      // (N) new -> old, or null (no renumbering)
    int n;
};

// Old index of new site i. perm is expected to be a permutation; an entry outside [0, N) is clamped so that no
// access leaves the arrays (the records are then meaningless, not out of bounds).
__device__ __forceinline__ int old_of(const PackIn& P, int i) {
    return P.perm != nullptr ? min(max(P.perm[i], 0), P.n - 1) : i;
}

// Per old site: (p, half2 cut-off word) as one float4, the edge record of every edge that ends at it, and
// inv[old] = new when renumbering.
__global__ void __launch_bounds__(kBlock)
    pack_cut_kernel(PackIn P, float floor2, float log_eps, int eps_on, float4* __restrict__ site4,
                    int* __restrict__ inv) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= P.n) return;
    float r2 = __builtin_huge_valf();
    if (eps_on) {
        float s_max2 = -kInf;
#pragma unroll
        for (int k = 0; k < 3; ++k)
            s_max2 = fmaxf(s_max2, expf(2.f * fminf(fmaxf(P.d_log_scale[3 * i + k], -20.f), 20.f)) + floor2);
        r2 = 2.f * s_max2 * fmaxf(fminf(P.raw[i], 30.f) - log_eps, 0.f) * (1.f + 0x1p-9f);
    }
    float c_max2 = -kInf;
#pragma unroll
    for (int k = 0; k < 3; ++k)
        c_max2 = fmaxf(c_max2, expf(2.f * fminf(fmaxf(P.c_log_scale[3 * i + k], -20.f), 20.f)) + floor2);
    const float lam = fminf(1.f / c_max2 * (1.f - 0x1p-9f), 65000.f);
    const uint16_t lo = __builtin_bit_cast(uint16_t, static_cast<_Float16>(r2));
    const uint16_t hi = __builtin_bit_cast(uint16_t, static_cast<_Float16>(lam));
    const uint32_t cut = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
    site4[i] = make_float4(P.points[3 * i], P.points[3 * i + 1], P.points[3 * i + 2], __uint_as_float(cut));
    if (P.perm != nullptr) inv[old_of(P, static_cast<int>(i))] = static_cast<int>(i);
}

// Self-first row size of new site i.
__global__ void __launch_bounds__(kBlock) pack_size_kernel(PackIn P, int* __restrict__ size) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= P.n) return;
    const int o = old_of(P, static_cast<int>(i));
    size[i] = P.offsets[o + 1] - P.offsets[o] + 1;
}

// Site records and positions of new site i.
__global__ void __launch_bounds__(kBlock)
    pack_sites_kernel(PackIn P, float4* __restrict__ pts4, float* __restrict__ attr) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= P.n) return;
    const int64_t o = old_of(P, static_cast<int>(i));
    pts4[i] = make_float4(P.points[3 * o], P.points[3 * o + 1], P.points[3 * o + 2], 0.f);
    float* a = attr + 20 * i;
#pragma unroll
    for (int k = 0; k < 6; ++k) a[k] = P.dA[6 * o + k];
    a[6] = fminf(P.raw[o], 30.f), a[7] = 0.f;
#pragma unroll
    for (int k = 0; k < 6; ++k) a[8 + k] = P.cA[6 * o + k];
#pragma unroll
    for (int k = 14; k < 20; ++k) a[k] = 0.f;
}

// SH rows in the new numbering, one float4 (of the 12 of a row) per lane, so that a wave writes 1 KB contiguously
// (fp32, and fp16 when sh16 is given).
__global__ void __launch_bounds__(kBlock)
    pack_sh_kernel(PackIn P, float4* __restrict__ sh32, uint2* __restrict__ sh16) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= 12 * static_cast<int64_t>(P.n)) return;
    const int64_t i = t / 12, q = t - 12 * i;
    const float4 f = P.sh[12 * static_cast<int64_t>(old_of(P, static_cast<int>(i))) + q];
    sh32[t] = f;
    if (sh16 != nullptr) {
        const uint32_t x = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f.x)),
                       y = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f.y)),
                       z = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f.z)),
                       w = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f.w));
        sh16[t] = make_uint2(x | (y << 16), z | (w << 16));
    }
}

// The self-first rows of new sites i0 .. i0 + 63 (one wave): each site itself, then its neighbours in CSR order,
// renumbered. The rows are contiguous in the output, so the wave walks them with one lane per output entry (every
// store contiguous across the wave); a lane finds the site of its entry by a binary search over the 64 row starts,
// which lane s holds for site i0 + s. All lanes run every step (the shuffles read any lane).
__global__ void __launch_bounds__(kBlock)
    pack_edges_kernel(PackIn P, const float4* __restrict__ site4, const int* __restrict__ inv,
                      const int* __restrict__ start, int* __restrict__ nbr, float4* __restrict__ edge) {
    const int lane = static_cast<int>(threadIdx.x) % 64;
    const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) / 64 * 64;
    if (i0 >= P.n) return;  // whole waves
    const int cnt = static_cast<int>(min(int64_t{64}, P.n - i0));
    const int64_t w_begin = start[i0], w_end = start[i0 + cnt];
    const bool has = lane < cnt;
    const int my_start = has ? start[i0 + lane] : static_cast<int>(w_end);  // past the rows: never <= an entry
    const int my_old = has ? old_of(P, static_cast<int>(i0 + lane)) : 0;
    const int my_e0 = has ? P.offsets[my_old] : 0;
    for (int64_t base = w_begin; base < w_end; base += 64) {
        const int64_t w = base + lane;
        int s = 0;  // the largest s with start[i0 + s] <= w
#pragma unroll
        for (int step = 32; step > 0; step >>= 1) {
            const int sm = __shfl(my_start, s + step);
            if (sm <= w) s += step;
        }
        const int row = __shfl(my_start, s), old = __shfl(my_old, s), e0 = __shfl(my_e0, s);
        if (w < w_end) {
            const int e = static_cast<int>(w - row);
            if (e == 0) {
                nbr[w] = static_cast<int>(i0 + s);
                edge[w] = site4[old];
            } else {
                const int j = P.adj[e0 + e - 1];
                nbr[w] = P.perm != nullptr ? inv[j] : j;
                edge[w] = site4[j];
            }
        }
    }
}

// Scratch: float4 site4[N], int inv[N], int size[N], int tile_sum[tiles + 1] (sections 256-byte aligned).
constexpr int64_t align256p(int64_t b) { return (b + 255) / 256 * 256; }

int64_t pack_bytes(int64_t n) {
    return align256p(16 * n) + 2 * align256p(4 * n) + align256p(4 * (scan_tiles_of(n) + 1));
}


__global__ void __launch_bounds__(kBlock)
    morton_kernel(const float* __restrict__ points, int64_t n, const float* __restrict__ box, int bits,
                  int64_t* __restrict__ code) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    const float scale = static_cast<float>((1 << bits) - 1);
    int64_t key = 0;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const float lo = box[a], ext = fmaxf(box[3 + a] - lo, 1e-12f);
        const int64_t q = static_cast<int64_t>((points[3 * i + a] - lo) / ext * scale);
        for (int b = 0; b < bits; ++b) key |= ((q >> b) & 1) << (3 * b + a);
    }
    code[i] = key;
}

// Baked colour of site i for the view from c = (cx, cy, cz) (render.py:228-235): max(SH_i(d) + 1/2, 0) with
// d = (p_i - c) / max(|p_i - c|, 1e-12), written to attr[20 i + 16 .. 18]. The basis is sh_basis's; the
// coefficients of degree <= deg are summed in storage order, and only their float4 are read.
__global__ void __launch_bounds__(kBlock)
    bake_kernel(const float4* __restrict__ points4, const float4* __restrict__ sh32, int64_t n, int deg, float cx,
                float cy, float cz, float* __restrict__ attr) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    const float4 p = points4[i];
    float dx = p.x - cx, dy = p.y - cy, dz = p.z - cz;
    const float nrm = fmaxf(sqrtf(dx * dx + dy * dy + dz * dz), 1e-12f);
    dx /= nrm, dy /= nrm, dz /= nrm;
    float b[16];
    sh_basis(dx, dy, dz, deg, b);
    const int nb = (deg + 1) * (deg + 1);
    float c[3] = {0.f, 0.f, 0.f};
    const float4* s = sh32 + 12 * i;
#pragma unroll
    for (int q = 0; q < 12; ++q) {
        if (4 * q >= 3 * nb) break;
        const float4 f = s[q];
        const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = 4 * q + u;
            if (j / 3 < nb) c[j % 3] += b[j / 3] * fv[u];
        }
    }
    float* a = attr + 20 * i;
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) a[16 + ch] = fmaxf(c[ch] + 0.5f, 0.f);
}

}  // namespace
}  // namespace vgr

extern "C" int vgr_bake_colors(const float* points4, const float* sh32, int64_t n_sites, int64_t sh_deg,
                               double cx, double cy, double cz, float* attr, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(n_sites >= 0, "bake_colors: n_sites must be >= 0");
    VGR_REQUIRE(sh_deg >= 0 && sh_deg <= 3, "sh_deg must be in [0, 3] (got %lld)", static_cast<long long>(sh_deg));
    if (n_sites == 0) return VGR_OK;
    VGR_REQUIRE(points4 && sh32 && attr, "bake_colors: null pointer");
    hipLaunchKernelGGL(bake_kernel, dim3(grid_for(n_sites, kBlock)), dim3(kBlock), 0, as_stream(stream),
                       reinterpret_cast<const float4*>(points4), reinterpret_cast<const float4*>(sh32), n_sites,
                       int(sh_deg), float(cx), float(cy), float(cz), attr);
    return launch_status("bake_kernel");
}

extern "C" int64_t vgr_morton_work_size(int64_t n) {
    return n > 0 ? 4 * 6 * vgr::grid_for(n, vgr::kBlock) : 0;
}

extern "C" int vgr_morton_codes(const float* points, int64_t n, int32_t bits, int64_t* code, void* work,
                                int64_t work_bytes, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(n >= 0, "morton_codes: n must be >= 0");
    VGR_REQUIRE(bits >= 1 && bits <= 21, "morton_codes: bits must be in [1, 21] (got %d)", bits);
    if (n == 0) return VGR_OK;
    VGR_REQUIRE(points && code, "morton_codes: null pointer");
    const int64_t blocks = grid_for(n, kBlock);
    VGR_REQUIRE(work != nullptr && work_bytes >= 4 * 6 * blocks, "morton_codes: work must hold %lld bytes",
                static_cast<long long>(4 * 6 * blocks));
    float* box = static_cast<float*>(work);
    const hipStream_t s = as_stream(stream);
    bounding_box(points, n, box, s);
    hipLaunchKernelGGL(morton_kernel, dim3(blocks), dim3(kBlock), 0, s, points, n, box, int(bits), code);
    return launch_status("morton_codes");
}

extern "C" int64_t vgr_pack_work_size(int64_t n_sites) { return n_sites > 0 ? vgr::pack_bytes(n_sites) : 0; }

extern "C" int vgr_pack_foam(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                             int64_t n_adj, const float* raw, const float* d_log_scale, const float* c_log_scale,
                             const float* dA, const float* cA, const float* sh, const int32_t* perm,
                             double scale_floor, double eps_density, float* points4, int32_t* offsets_sf,
                             int32_t* nbr, float* edge, float* attr, float* sh32, void* sh16, void* work,
                             int64_t work_bytes, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(n_sites > 0 && n_sites <= int64_t(kScanTile) * kScanTile,
                "pack_foam: n_sites must be in [1, %lld]", static_cast<long long>(int64_t(kScanTile) * kScanTile));
    VGR_REQUIRE(n_adj >= 0 && n_adj + n_sites <= INT_MAX, "pack_foam: n_adj + n_sites must be < 2^31");
    VGR_REQUIRE(points && offsets && (adj || n_adj == 0) && raw && d_log_scale && c_log_scale && dA && cA && sh,
                "pack_foam: null input pointer");
    VGR_REQUIRE(points4 && offsets_sf && nbr && edge && attr && sh32, "pack_foam: null output pointer");
    VGR_REQUIRE(eps_density >= 0.0, "pack_foam: eps_density must be >= 0");
    VGR_REQUIRE(work != nullptr && work_bytes >= pack_bytes(n_sites) && reinterpret_cast<uintptr_t>(work) % 256 == 0,
                "pack_foam: work must hold vgr_pack_work_size(N) = %lld bytes, 256-byte aligned",
                static_cast<long long>(pack_bytes(n_sites)));
    const PackIn P{points, offsets, adj, raw, d_log_scale, c_log_scale, dA, cA, reinterpret_cast<const float4*>(sh),
                   perm, int(n_sites)};
    char* w = static_cast<char*>(work);
    float4* site4 = reinterpret_cast<float4*>(w);
    w += align256p(16 * n_sites);
    int* inv = reinterpret_cast<int*>(w);
    w += align256p(4 * n_sites);
    int* size = reinterpret_cast<int*>(w);
    w += align256p(4 * n_sites);
    int* tile_sum = reinterpret_cast<int*>(w);
    const hipStream_t s = as_stream(stream);
    const dim3 grid(grid_for(n_sites, kBlock)), block(kBlock);
    // ln(eps) in double, then fp32, as a Python float meets a float32 tensor
    const float log_eps = eps_density > 0.0 ? static_cast<float>(std::log(eps_density)) : 0.f;
    hipLaunchKernelGGL(pack_cut_kernel, grid, block, 0, s, P, static_cast<float>(scale_floor * scale_floor), log_eps,
                       eps_density > 0.0 ? 1 : 0, site4, inv);
    hipLaunchKernelGGL(pack_size_kernel, grid, block, 0, s, P, size);
    exclusive_scan(size, n_sites, offsets_sf, size, tile_sum, s);  // offsets_sf[0 .. N]
    hipLaunchKernelGGL(pack_sites_kernel, grid, block, 0, s, P, reinterpret_cast<float4*>(points4), attr);
    hipLaunchKernelGGL(pack_sh_kernel, dim3(grid_for(12 * n_sites, kBlock)), block, 0, s, P,
                       reinterpret_cast<float4*>(sh32), static_cast<uint2*>(sh16));
    hipLaunchKernelGGL(pack_edges_kernel, grid, block, 0, s, P, site4, inv, offsets_sf, nbr,
                       reinterpret_cast<float4*>(edge));
    return launch_status("pack_foam");
}
