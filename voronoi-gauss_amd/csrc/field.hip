// Forward field operators of the NeRF-style path, gfx950: greedy walk of sorted samples, density and colour
// at samples over the Voronoi neighbourhood, and conics from (log_scale, quat).
//
// Semantics follow csrc/vgf.cu of the reference: walk_kernel :51-79 (strict <, so the first closer neighbour
// in CSR order wins), gauss_local :98-119 and density_forward_kernel :163-177, sh_eval/unit_dir/
// color_forward_kernel :230-282 (online softmax), conic_local/conic_forward_kernel :350-380.
// One work item (ray, sample or site) per lane, 256-lane workgroups; all loops are over <= ~60 neighbours.
#include "vgr_abi.h"
#include "vgr_device.h"

namespace vgr {
namespace {

constexpr int kBlock = 256;

struct Graph {
    const float* __restrict__ points;  // (N, 3)
    const int* __restrict__ offsets;   // (N + 1)
    const int* __restrict__ adj;       // (M)
    int n_sites;
};

struct Gauss {
    const float* __restrict__ log_scale;  // (N, 3)
    const float4* __restrict__ quat;      // (N) w x y z, not normalised
};

__device__ __forceinline__ float dist2(const float* __restrict__ p, int i, float x, float y, float z) {
    const float dx = x - p[3 * static_cast<int64_t>(i)], dy = y - p[3 * static_cast<int64_t>(i) + 1],
                dz = z - p[3 * static_cast<int64_t>(i) + 2];
    return dx * dx + dy * dy + dz * dz;
}

__global__ void __launch_bounds__(kBlock)
    walk_kernel(Graph g, const float* __restrict__ o, const float* __restrict__ d, const float* __restrict__ z,
                const int* __restrict__ start, int64_t B, int S, int* __restrict__ site, int* __restrict__ steps) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (r >= B) return;
    const float ox = o[3 * r], oy = o[3 * r + 1], oz = o[3 * r + 2];
    const float dx = d[3 * r], dy = d[3 * r + 1], dz = d[3 * r + 2];
    int cur = start[r];
    if (cur < 0 || cur >= g.n_sites) {  // invalid start: every sample unresolved
        for (int s = 0; s < S; ++s) site[r * S + s] = -1;
        if (steps != nullptr) steps[r] = 0;
        return;
    }
    int total = 0;
    for (int s = 0; s < S; ++s) {
        const float t = z[r * S + s];
        const float x = ox + t * dx, y = oy + t * dy, w = oz + t * dz;
        float best_d = dist2(g.points, cur, x, y, w);
        for (int it = 0; it < kWalkCap; ++it) {
            int best = cur;
            const int e1 = g.offsets[cur + 1];
            for (int e = g.offsets[cur]; e < e1; ++e) {
                const int q = g.adj[e];
                const float dq = dist2(g.points, q, x, y, w);
                if (dq < best_d) best_d = dq, best = q;
            }
            if (best == cur) break;
            cur = best;
            ++total;
        }
        site[r * S + s] = cur;
    }
    if (steps != nullptr) steps[r] = total;
}

// Mahalanobis distance of (x, y, z) to Gaussian i, with the inverse variances scaled by inv_mult2.
__device__ __forceinline__ float gauss_m(const Graph& g, const Gauss& G, int i, float x, float y, float z,
                                         float inv_mult2) {
    const int64_t i3 = 3 * static_cast<int64_t>(i);
    const float v0 = x - g.points[i3], v1 = y - g.points[i3 + 1], v2 = z - g.points[i3 + 2];
    const float4 q = G.quat[i];
    const float qnorm = fmaxf(sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w), 1e-12f);
    const float w = q.x / qnorm, a = q.y / qnorm, b = q.z / qnorm, c = q.w / qnorm;
    const float R[9] = {1.f - 2.f * (b * b + c * c), 2.f * (a * b - w * c),       2.f * (a * c + w * b),
                        2.f * (a * b + w * c),       1.f - 2.f * (a * a + c * c), 2.f * (b * c - w * a),
                        2.f * (a * c - w * b),       2.f * (b * c + w * a),       1.f - 2.f * (a * a + b * b)};
    float m = 0.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const float yk = R[k] * v0 + R[3 + k] * v1 + R[6 + k] * v2;
        const float s = fexp(fminf(fmaxf(G.log_scale[i3 + k], -20.f), 20.f));
        const float is2 = inv_mult2 / (s * s);
        m += yk * yk * is2;
    }
    return m;
}

// Per-site Gaussian records, built once per call by gauss_pack_kernel with gauss_m's own arithmetic, so that the
// per-neighbour work is the rotation and the sum only: rec[4i .. 4i + 2] = rows of R with the inverse variances
// (R0, R1, R2, is2_0), (R3, R4, R5, is2_1), (R6, R7, R8, is2_2); rec[4i + 3] = (p_i, min(raw_i, 30)) (0 without raw).
// gauss_m rebuilds R from the quaternion (four divisions, a square root) and takes three exponentials and three
// more divisions for every neighbour of every sample; a call with m samples over N sites does that m E / N times
// per site.
constexpr int kGRec = 4;

__global__ void __launch_bounds__(kBlock)
    gauss_pack_kernel(Graph g, Gauss G, const float* __restrict__ raw, float inv_mult2, float4* __restrict__ rec) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= g.n_sites) return;
    const float4 q = G.quat[i];
    const float qnorm = fmaxf(sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w), 1e-12f);
    const float w = q.x / qnorm, a = q.y / qnorm, b = q.z / qnorm, c = q.w / qnorm;
    const float R[9] = {1.f - 2.f * (b * b + c * c), 2.f * (a * b - w * c),       2.f * (a * c + w * b),
                        2.f * (a * b + w * c),       1.f - 2.f * (a * a + c * c), 2.f * (b * c - w * a),
                        2.f * (a * c - w * b),       2.f * (b * c + w * a),       1.f - 2.f * (a * a + b * b)};
    float is2[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const float s = fexp(fminf(fmaxf(G.log_scale[3 * i + k], -20.f), 20.f));
        is2[k] = inv_mult2 / (s * s);
    }
    float4* r = rec + kGRec * i;
    r[0] = make_float4(R[0], R[1], R[2], is2[0]);
    r[1] = make_float4(R[3], R[4], R[5], is2[1]);
    r[2] = make_float4(R[6], R[7], R[8], is2[2]);
    r[3] = make_float4(g.points[3 * i], g.points[3 * i + 1], g.points[3 * i + 2],
                       raw != nullptr ? fminf(raw[i], 30.f) : 0.f);
}

// gauss_m of site i from its record; raw_c = min(raw_i, 30).
__device__ __forceinline__ float gauss_m_rec(const float4* __restrict__ rec, int i, float x, float y, float z,
                                             float& raw_c) {
    const float4* r = rec + kGRec * static_cast<int64_t>(i);
    const float4 r0 = r[0], r1 = r[1], r2 = r[2], r3 = r[3];
    const float v0 = x - r3.x, v1 = y - r3.y, v2 = z - r3.z;
    const float c0[3] = {r0.x, r0.y, r0.z}, c1[3] = {r1.x, r1.y, r1.z}, c2[3] = {r2.x, r2.y, r2.z};
    const float is2[3] = {r0.w, r1.w, r2.w};
    float m = 0.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const float yk = c0[k] * v0 + c1[k] * v1 + c2[k] * v2;
        m += yk * yk * is2[k];
    }
    raw_c = r3.w;
    return m;
}

__global__ void __launch_bounds__(kBlock)
    density_forward_packed_kernel(Graph g, const float4* __restrict__ rec, const float* __restrict__ x,
                                  const int* __restrict__ site, int64_t m, float* __restrict__ sigma) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= m) return;
    const float qx = x[3 * t], qy = x[3 * t + 1], qz = x[3 * t + 2];
    const int i = site[t];
    if (i < 0 || i >= g.n_sites) {
        sigma[t] = 0.f;
        return;
    }
    float s = 0.f;
    const int e0 = g.offsets[i], e1 = g.offsets[i + 1];
    for (int e = e0 - 1; e < e1; ++e) {
        const int k = e < e0 ? i : g.adj[e];
        float raw_c;
        const float mk = gauss_m_rec(rec, k, qx, qy, qz, raw_c);
        s += fexp(raw_c - 0.5f * mk);
    }
    sigma[t] = s;
}

__global__ void __launch_bounds__(kBlock)
    density_forward_kernel(Graph g, const float* __restrict__ raw, Gauss G, const float* __restrict__ x,
                           const int* __restrict__ site, int64_t m, float inv_mult2, float* __restrict__ sigma) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= m) return;
    const float qx = x[3 * t], qy = x[3 * t + 1], qz = x[3 * t + 2];
    const int i = site[t];
    if (i < 0 || i >= g.n_sites) {
        sigma[t] = 0.f;
        return;
    }
    float s = 0.f;
    const int e0 = g.offsets[i], e1 = g.offsets[i + 1];
    for (int e = e0 - 1; e < e1; ++e) {
        const int k = e < e0 ? i : g.adj[e];
        s += fexp(fminf(raw[k], 30.f) - 0.5f * gauss_m(g, G, k, qx, qy, qz, inv_mult2));
    }
    sigma[t] = s;
}

template <int NV>
__device__ __forceinline__ void sh_eval_n(const float4* __restrict__ sh, int k, const float (&b)[16], int nb,
                                          float (&c)[3]) {
    const float4* s = sh + 12 * static_cast<int64_t>(k);
    c[0] = c[1] = c[2] = 0.5f;
#pragma unroll
    for (int q = 0; q < NV; ++q) {
        const float4 f = s[q];
        const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = 4 * q + u;
            if (i / 3 < nb) c[i % 3] += b[i / 3] * fv[u];
        }
    }
}

template <int DEG>
__global__ void __launch_bounds__(kBlock)
    color_forward_kernel(Graph g, Gauss H, const float4* __restrict__ sh, const float* __restrict__ x,
                         const float* __restrict__ dirs, const int* __restrict__ site, int64_t m,
                         float* __restrict__ rgb) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= m) return;
    const int i = site[t];
    if (i < 0 || i >= g.n_sites) {
        rgb[3 * t] = rgb[3 * t + 1] = rgb[3 * t + 2] = 0.f;
        return;
    }
    const float qx = x[3 * t], qy = x[3 * t + 1], qz = x[3 * t + 2];
    float dx = dirs[3 * t], dy = dirs[3 * t + 1], dz = dirs[3 * t + 2];
    const float inv = rsqrtf(fmaxf(dx * dx + dy * dy + dz * dz, 1e-20f));
    dx *= inv, dy *= inv, dz *= inv;
    float b[16];
    sh_basis(dx, dy, dz, DEG, b);
    constexpr int nb = (DEG + 1) * (DEG + 1);
    float mmin = kInf, A = 0.f, cr = 0.f, cg = 0.f, cb = 0.f;
    const int e0 = g.offsets[i], e1 = g.offsets[i + 1];
    for (int e = e0 - 1; e < e1; ++e) {
        const int k = e < e0 ? i : g.adj[e];
        const float mk = gauss_m(g, H, k, qx, qy, qz, 1.f);
        if (mk < mmin) {
            const float f = mmin == kInf ? 0.f : fexp(-0.5f * (mmin - mk));
            A *= f, cr *= f, cg *= f, cb *= f;
            mmin = mk;
        }
        const float a = fexp(-0.5f * (mk - mmin));
        float c[3];
        sh_eval_n<sh_vec4_f32(DEG)>(sh, k, b, nb, c);
        A += a;
        cr += a * fmaxf(c[0], 0.f);
        cg += a * fmaxf(c[1], 0.f);
        cb += a * fmaxf(c[2], 0.f);
    }
    rgb[3 * t] = cr / A;
    rgb[3 * t + 1] = cg / A;
    rgb[3 * t + 2] = cb / A;
}

template <int DEG>
__global__ void __launch_bounds__(kBlock)
    color_forward_packed_kernel(Graph g, const float4* __restrict__ rec, const float4* __restrict__ sh,
                                const float* __restrict__ x, const float* __restrict__ dirs,
                                const int* __restrict__ site, int64_t m, float* __restrict__ rgb) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= m) return;
    const int i = site[t];
    if (i < 0 || i >= g.n_sites) {
        rgb[3 * t] = rgb[3 * t + 1] = rgb[3 * t + 2] = 0.f;
        return;
    }
    const float qx = x[3 * t], qy = x[3 * t + 1], qz = x[3 * t + 2];
    float dx = dirs[3 * t], dy = dirs[3 * t + 1], dz = dirs[3 * t + 2];
    const float inv = rsqrtf(fmaxf(dx * dx + dy * dy + dz * dz, 1e-20f));
    dx *= inv, dy *= inv, dz *= inv;
    float b[16];
    sh_basis(dx, dy, dz, DEG, b);
    constexpr int nb = (DEG + 1) * (DEG + 1);
    float mmin = kInf, A = 0.f, cr = 0.f, cg = 0.f, cb = 0.f;
    const int e0 = g.offsets[i], e1 = g.offsets[i + 1];
    for (int e = e0 - 1; e < e1; ++e) {
        const int k = e < e0 ? i : g.adj[e];
        float raw_c;
        const float mk = gauss_m_rec(rec, k, qx, qy, qz, raw_c);
        if (mk < mmin) {
            const float f = mmin == kInf ? 0.f : fexp(-0.5f * (mmin - mk));
            A *= f, cr *= f, cg *= f, cb *= f;
            mmin = mk;
        }
        const float a = fexp(-0.5f * (mk - mmin));
        float c[3];
        sh_eval_n<sh_vec4_f32(DEG)>(sh, k, b, nb, c);
        A += a;
        cr += a * fmaxf(c[0], 0.f);
        cg += a * fmaxf(c[1], 0.f);
        cb += a * fmaxf(c[2], 0.f);
    }
    rgb[3 * t] = cr / A;
    rgb[3 * t + 1] = cg / A;
    rgb[3 * t + 2] = cb / A;
}

__global__ void __launch_bounds__(kBlock)
    conic_forward_kernel(const float* __restrict__ log_scale, const float4* __restrict__ quat, int64_t n,
                         float floor2, float* __restrict__ A) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    const float4 q = quat[i];
    const float qnorm = fmaxf(sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w), 1e-12f);
    const float w = q.x / qnorm, a = q.y / qnorm, b = q.z / qnorm, c = q.w / qnorm;
    const float R[9] = {1.f - 2.f * (b * b + c * c), 2.f * (a * b - w * c),       2.f * (a * c + w * b),
                        2.f * (a * b + w * c),       1.f - 2.f * (a * a + c * c), 2.f * (b * c - w * a),
                        2.f * (a * c - w * b),       2.f * (b * c + w * a),       1.f - 2.f * (a * a + b * b)};
    float iv[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const float s = fexp(2.f * fminf(fmaxf(log_scale[3 * i + k], -20.f), 20.f));
        iv[k] = 1.f / (s + floor2);
    }
    constexpr int ab[6][2] = {{0, 0}, {0, 1}, {0, 2}, {1, 1}, {1, 2}, {2, 2}};
#pragma unroll
    for (int e = 0; e < 6; ++e) {
        const int p = ab[e][0], q2 = ab[e][1];
        A[6 * i + e] = R[3 * p] * R[3 * q2] * iv[0] + R[3 * p + 1] * R[3 * q2 + 1] * iv[1] +
                       R[3 * p + 2] * R[3 * q2 + 2] * iv[2];
    }
}

// The records pay for themselves once a call has about N / 8 samples (their build reads and writes each site once;
// the gauss_m work they remove is per neighbour of every sample); both paths give the same bits.
bool use_records(const void* work, int64_t work_bytes, int64_t n_sites, int64_t m) {
    return work != nullptr && work_bytes >= n_sites * kGRec * static_cast<int64_t>(sizeof(float4)) &&
           reinterpret_cast<uintptr_t>(work) % 16 == 0 && m * 8 >= n_sites;
}

int check_graph(const char* op, const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                int64_t n_adj) {
    VGR_REQUIRE(n_sites > 0 && n_sites <= INT_MAX, "%s: n_sites must be in [1, 2^31)", op);
    VGR_REQUIRE(n_adj >= 0 && n_adj <= INT_MAX, "%s: n_adj must be in [0, 2^31)", op);
    VGR_REQUIRE(points && offsets && (adj || n_adj == 0), "%s: null graph pointer", op);
    return VGR_OK;
}

}  // namespace
}  // namespace vgr

extern "C" int64_t vgr_field_work_size(int64_t n_sites) {
    return n_sites > 0 ? n_sites * vgr::kGRec * static_cast<int64_t>(sizeof(float4)) : 0;
}

extern "C" int vgr_walk(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                        int64_t n_adj, const float* o, const float* d, const float* z, const int32_t* start,
                        int64_t n_rays, int64_t n_samples, int32_t* site, int32_t* steps, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(n_rays >= 0 && n_samples >= 0 && n_samples <= INT_MAX, "walk: bad sizes");
    if (n_rays == 0) return VGR_OK;
    if (int rc = check_graph("walk", points, n_sites, offsets, adj, n_adj)) return rc;
    VGR_REQUIRE(o && d && start && site && (z || n_samples == 0), "walk: null pointer");
    hipLaunchKernelGGL(walk_kernel, dim3(grid_for(n_rays, kBlock)), dim3(kBlock), 0, as_stream(stream),
                       Graph{points, offsets, adj, int(n_sites)}, o, d, z, start, n_rays, int(n_samples), site, steps);
    return launch_status("walk_kernel");
}

extern "C" int vgr_density_forward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                                   int64_t n_adj, const float* raw, const float* log_scale, const float* quat,
                                   const float* x, const int32_t* site, int64_t m, double scale_mult, float* sigma,
                                   void* work, int64_t work_bytes, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(m >= 0, "density_forward: m must be >= 0");
    if (m == 0) return VGR_OK;
    if (int rc = check_graph("density_forward", points, n_sites, offsets, adj, n_adj)) return rc;
    VGR_REQUIRE(raw && log_scale && quat && x && site && sigma, "density_forward: null pointer");
    VGR_REQUIRE(scale_mult != 0.0, "density_forward: scale_mult must be non-zero");
    const float inv_mult2 = static_cast<float>(1.0 / (scale_mult * scale_mult));
    const Graph g{points, offsets, adj, int(n_sites)};
    const Gauss G{log_scale, reinterpret_cast<const float4*>(quat)};
    if (use_records(work, work_bytes, n_sites, m)) {
        float4* rec = static_cast<float4*>(work);
        hipLaunchKernelGGL(gauss_pack_kernel, dim3(grid_for(n_sites, kBlock)), dim3(kBlock), 0, as_stream(stream), g,
                           G, raw, inv_mult2, rec);
        hipLaunchKernelGGL(density_forward_packed_kernel, dim3(grid_for(m, kBlock)), dim3(kBlock), 0,
                           as_stream(stream), g, rec, x, site, m, sigma);
        return launch_status("density_forward_packed_kernel");
    }
    hipLaunchKernelGGL(density_forward_kernel, dim3(grid_for(m, kBlock)), dim3(kBlock), 0, as_stream(stream), g, raw, G,
                       x, site, m, inv_mult2, sigma);
    return launch_status("density_forward_kernel");
}

extern "C" int vgr_color_forward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                                 int64_t n_adj, const float* log_scale, const float* quat, const float* sh,
                                 int64_t sh_deg, const float* x, const float* dirs, const int32_t* site, int64_t m,
                                 float* rgb, void* work, int64_t work_bytes, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(m >= 0, "color_forward: m must be >= 0");
    VGR_REQUIRE(sh_deg >= 0 && sh_deg <= 3, "sh_deg must be in [0, 3] (got %lld)", static_cast<long long>(sh_deg));
    if (m == 0) return VGR_OK;
    if (int rc = check_graph("color_forward", points, n_sites, offsets, adj, n_adj)) return rc;
    VGR_REQUIRE(log_scale && quat && sh && x && dirs && site && rgb, "color_forward: null pointer");
    const Graph g{points, offsets, adj, int(n_sites)};
    const Gauss H{log_scale, reinterpret_cast<const float4*>(quat)};
    const float4* s4 = reinterpret_cast<const float4*>(sh);
    const dim3 grid(grid_for(m, kBlock)), block(kBlock);
    const hipStream_t st = as_stream(stream);
    if (use_records(work, work_bytes, n_sites, m)) {
        const float4* rec = static_cast<const float4*>(work);
        hipLaunchKernelGGL(gauss_pack_kernel, dim3(grid_for(n_sites, kBlock)), block, 0, st, g, H, nullptr, 1.f,
                           static_cast<float4*>(work));
        switch (sh_deg) {
            case 0: hipLaunchKernelGGL(color_forward_packed_kernel<0>, grid, block, 0, st, g, rec, s4, x, dirs, site, m,
                                       rgb); break;
            case 1: hipLaunchKernelGGL(color_forward_packed_kernel<1>, grid, block, 0, st, g, rec, s4, x, dirs, site, m,
                                       rgb); break;
            case 2: hipLaunchKernelGGL(color_forward_packed_kernel<2>, grid, block, 0, st, g, rec, s4, x, dirs, site, m,
                                       rgb); break;
            default: hipLaunchKernelGGL(color_forward_packed_kernel<3>, grid, block, 0, st, g, rec, s4, x, dirs, site,
                                        m, rgb); break;
        }
        return launch_status("color_forward_packed_kernel");
    }
    switch (sh_deg) {
        case 0: hipLaunchKernelGGL(color_forward_kernel<0>, grid, block, 0, st, g, H, s4, x, dirs, site, m, rgb); break;
        case 1: hipLaunchKernelGGL(color_forward_kernel<1>, grid, block, 0, st, g, H, s4, x, dirs, site, m, rgb); break;
        case 2: hipLaunchKernelGGL(color_forward_kernel<2>, grid, block, 0, st, g, H, s4, x, dirs, site, m, rgb); break;
        default:
            hipLaunchKernelGGL(color_forward_kernel<3>, grid, block, 0, st, g, H, s4, x, dirs, site, m, rgb);
            break;
    }
    return launch_status("color_forward_kernel");
}

extern "C" int vgr_conic_forward(const float* log_scale, const float* quat, int64_t n, double floor, float* A,
                                 void* stream) {
    using namespace vgr;
    VGR_REQUIRE(n >= 0, "conic_forward: n must be >= 0");
    if (n == 0) return VGR_OK;
    VGR_REQUIRE(log_scale && quat && A, "conic_forward: null pointer");
    hipLaunchKernelGGL(conic_forward_kernel, dim3(grid_for(n, kBlock)), dim3(kBlock), 0, as_stream(stream),
                       log_scale, reinterpret_cast<const float4*>(quat), n, static_cast<float>(floor * floor), A);
    return launch_status("conic_forward_kernel");
}
