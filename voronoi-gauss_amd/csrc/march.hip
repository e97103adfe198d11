// Fused uniform-step march (forward), gfx950.
//
// Semantics follow csrc/march.cu:134-262 of the reference: midpoints of dt steps from near to the unit-sphere
// exit `mid`, then n_bg steps uniform in disparity out to `far`; at every sample a greedy walk to the
// nearest site (lexicographic (distance, index) argmin over the Delaunay neighbourhood), the density sum,
// NeRF compositing alpha = 1 - exp(-sigma delta), and the two-pass normalised colour blend for samples with
// weight > w_thresh; the ray stops once T < t_thresh.
//
// MI355X mapping: one ray per lane over 8x8 ray tiles. All lanes of a wave sit at the same sample index k
// (the step grid is shared), adjacent pixels are at nearby points, so the neighbourhood gathers of a wave
// mostly hit the same sites (one broadcast line instead of 64 random ones). The reference's 32-lane
// shuffle reductions become sequential per-lane sums.
#include "vgr_abi.h"
#include "vgr_device.h"

namespace vgr {
namespace {

constexpr int kBlock = 64;

struct MarchField {
    const float* __restrict__ points;  // (N, 3)
    const int* __restrict__ offsets;   // (N + 1)
    const int* __restrict__ adj;       // (M)
    const float* __restrict__ raw;     // (N)
    const float* __restrict__ dA;      // (N, 6)
    const float* __restrict__ cA;      // (N, 6)
    const float4* __restrict__ sh;     // (N, 12)
    int sh_deg, n_sites;
};

struct MarchParams {
    float dt;
    int n_bg;
    float t_thresh, w_thresh;
};

struct MarchRays {
    const float* __restrict__ o;
    const float* __restrict__ d;
    const int* __restrict__ start;
    const float* __restrict__ t_near;
    const float* __restrict__ t_mid;
    const float* __restrict__ t_far;
    int64_t n;
};

struct MarchOut {
    float* __restrict__ rgb;
    float* __restrict__ T;
    float* __restrict__ depth;
    int* __restrict__ stats;
    int* __restrict__ trace;
    int64_t trace_cap;
};

__device__ __forceinline__ int neighbor(const MarchField& F, int i, int e0, int e) {
    return e == 0 ? i : F.adj[e0 + e - 1];
}

__device__ __forceinline__ void offset_to(const MarchField& F, int k, const float (&x)[3], float (&v)[3]) {
    const float* p = F.points + 3 * static_cast<int64_t>(k);
    v[0] = x[0] - p[0], v[1] = x[1] - p[1], v[2] = x[2] - p[2];
}

__device__ __forceinline__ float conic_m(const float* __restrict__ A, int k, const float (&v)[3]) {
    const float* a = A + 6 * static_cast<int64_t>(k);
    return a[0] * v[0] * v[0] + a[3] * v[1] * v[1] + a[5] * v[2] * v[2] +
           2.f * (a[1] * v[0] * v[1] + a[2] * v[0] * v[2] + a[4] * v[1] * v[2]);
}

// 1/2 + sum_{j < (deg+1)^2} b_j sh_kj per channel, reading only the float4 that hold those coefficients.
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

__device__ __forceinline__ void sh_eval(const MarchField& F, int k, const float (&b)[16], int nb, float (&c)[3]) {
    switch (F.sh_deg) {
        case 0: sh_eval_n<sh_vec4_f32(0)>(F.sh, k, b, nb, c); break;
        case 1: sh_eval_n<sh_vec4_f32(1)>(F.sh, k, b, nb, c); break;
        case 2: sh_eval_n<sh_vec4_f32(2)>(F.sh, k, b, nb, c); break;
        default: sh_eval_n<sh_vec4_f32(3)>(F.sh, k, b, nb, c); break;
    }
}

__device__ __forceinline__ void sample_at(float near, float mid, float far, int n_in, const MarchParams& M, int k,
                                          float& t, float& delta) {
    if (k < n_in) {
        const float t0 = near + static_cast<float>(k) * M.dt, t1 = fminf(t0 + M.dt, mid);
        t = 0.5f * (t0 + t1), delta = t1 - t0;
    } else {
        const float i0 = 1.f / mid, i1 = 1.f / far;
        const float u0 = static_cast<float>(k - n_in) / static_cast<float>(M.n_bg);
        const float u1 = static_cast<float>(k - n_in + 1) / static_cast<float>(M.n_bg);
        t = 1.f / (i0 + 0.5f * (u0 + u1) * (i1 - i0));
        delta = 1.f / (i0 + u1 * (i1 - i0)) - 1.f / (i0 + u0 * (i1 - i0));
    }
}

// Lexicographic argmin of (|x - p|^2, index) over {cur} U adj(cur), repeated until cur wins.
__device__ int walk_to(const MarchField& F, int cur, const float (&x)[3], int& steps) {
    for (int it = 0; it < kWalkCap; ++it) {
        const int e0 = F.offsets[cur], n = F.offsets[cur + 1] - e0 + 1;
        float bd = kInf;
        int bk = INT_MAX;
        for (int e = 0; e < n; ++e) {
            const int k = neighbor(F, cur, e0, e);
            float v[3];
            offset_to(F, k, x, v);
            const float dk = v[0] * v[0] + v[1] * v[1] + v[2] * v[2];
            if (dk < bd || (dk == bd && k < bk)) bd = dk, bk = k;
        }
        if (bk == cur) break;
        cur = bk;
        ++steps;
    }
    return cur;
}

__device__ float density_at(const MarchField& F, int i, const float (&x)[3]) {
    const int e0 = F.offsets[i], n = F.offsets[i + 1] - e0 + 1;
    float s = 0.f;
    for (int e = 0; e < n; ++e) {
        const int k = neighbor(F, i, e0, e);
        float v[3];
        offset_to(F, k, x, v);
        s += fexp(fminf(F.raw[k], 30.f) - 0.5f * conic_m(F.dA, k, v));
    }
    return s;
}

__device__ void color_at(const MarchField& F, int i, const float (&x)[3], const float (&b)[16], float (&C)[3]) {
    const int e0 = F.offsets[i], n = F.offsets[i + 1] - e0 + 1;
    const int nb = (F.sh_deg + 1) * (F.sh_deg + 1);
    float mmin = kInf;
    for (int e = 0; e < n; ++e) {
        const int k = neighbor(F, i, e0, e);
        float v[3];
        offset_to(F, k, x, v);
        mmin = fminf(mmin, conic_m(F.cA, k, v));
    }
    float A = 0.f, cr = 0.f, cg = 0.f, cb = 0.f;
    for (int e = 0; e < n; ++e) {
        const int k = neighbor(F, i, e0, e);
        float v[3];
        offset_to(F, k, x, v);
        const float a = fexp(-0.5f * (conic_m(F.cA, k, v) - mmin));
        float c[3];
        sh_eval(F, k, b, nb, c);
        A += a, cr += a * fmaxf(c[0], 0.f), cg += a * fmaxf(c[1], 0.f), cb += a * fmaxf(c[2], 0.f);
    }
    const float inv_a = 1.f / A;
    C[0] = cr * inv_a, C[1] = cg * inv_a, C[2] = cb * inv_a;
}

template <bool TRACE>
__global__ void __launch_bounds__(kBlock)
    march_forward_kernel(MarchField F, MarchParams M, MarchRays R, MarchOut O) {
    const int64_t r = xcd_block_id() * kBlock + threadIdx.x;
    if (r >= R.n) return;
    int cur = R.start[r];
    if (cur < 0 || cur >= F.n_sites) {  // not traced: empty foreground
        O.rgb[3 * r] = O.rgb[3 * r + 1] = O.rgb[3 * r + 2] = 0.f;
        O.T[r] = 1.f, O.depth[r] = 0.f;
        O.stats[3 * r] = O.stats[3 * r + 1] = O.stats[3 * r + 2] = 0;
        return;
    }
    const float o[3] = {R.o[3 * r], R.o[3 * r + 1], R.o[3 * r + 2]};
    const float d[3] = {R.d[3 * r], R.d[3 * r + 1], R.d[3 * r + 2]};
    const float near = R.t_near[r], mid = R.t_mid[r], far = R.t_far[r];
    const int n_in = mid > near ? static_cast<int>(ceilf((mid - near) / M.dt)) : 0;
    const int n_total = n_in + M.n_bg;
    float b[16];
    sh_basis(d[0], d[1], d[2], F.sh_deg, b);
    int n_samples = 0, n_color = 0, walk_steps = 0;
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f}, dep = 0.f;
    for (int k = 0; k < n_total; ++k) {
        float t, delta, x[3];
        sample_at(near, mid, far, n_in, M, k, t, delta);
#pragma unroll
        for (int a = 0; a < 3; ++a) x[a] = o[a] + t * d[a];
        cur = walk_to(F, cur, x, walk_steps);
        if (TRACE && n_samples < O.trace_cap) O.trace[r * O.trace_cap + n_samples] = cur;
        const float alpha = 1.f - fexp(-density_at(F, cur, x) * delta);
        const float w = T * alpha;
        ++n_samples;
        if (w > M.w_thresh) {
            float C[3];
            color_at(F, cur, x, b, C);
#pragma unroll
            for (int a = 0; a < 3; ++a) acc[a] += w * C[a];
            dep += w * t;
            ++n_color;
        }
        T *= 1.f - alpha;
        if (T < M.t_thresh) break;
    }
#pragma unroll
    for (int a = 0; a < 3; ++a) O.rgb[3 * r + a] = acc[a];
    O.T[r] = T;
    O.depth[r] = dep;
    O.stats[3 * r] = n_samples, O.stats[3 * r + 1] = n_color, O.stats[3 * r + 2] = walk_steps;
}

}  // namespace
}  // namespace vgr

extern "C" int vgr_march_forward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                                 int64_t n_adj, const float* raw, const float* dA, const float* cA, const float* sh,
                                 int64_t sh_deg, const float* o, const float* d, const int32_t* start,
                                 const float* near_t, const float* mid_t, const float* far_t, int64_t n_rays,
                                 double dt, int64_t n_bg, double t_thresh, double w_thresh, float* rgb, float* T,
                                 float* depth, int32_t* stats, int32_t* trace, int64_t trace_cap, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(n_rays >= 0, "march_forward: n_rays must be >= 0 (got %lld)", static_cast<long long>(n_rays));
    VGR_REQUIRE(sh_deg >= 0 && sh_deg <= 3, "sh_deg must be in [0, 3] (got %lld)", static_cast<long long>(sh_deg));
    VGR_REQUIRE(n_bg >= 0 && n_bg <= INT_MAX, "march_forward: n_bg must be >= 0");
    VGR_REQUIRE(dt > 0.0, "march_forward: dt must be > 0");
    VGR_REQUIRE(trace == nullptr || trace_cap > 0, "march_forward: trace needs trace_cap > 0");
    if (n_rays == 0) return VGR_OK;
    VGR_REQUIRE(n_sites > 0 && n_sites <= INT_MAX, "march_forward: n_sites must be in [1, 2^31)");
    VGR_REQUIRE(n_adj >= 0 && n_adj <= INT_MAX, "march_forward: n_adj must be in [0, 2^31)");
    VGR_REQUIRE(points && offsets && (adj || n_adj == 0) && raw && dA && cA && sh, "march_forward: null field pointer");
    VGR_REQUIRE(o && d && start && near_t && mid_t && far_t, "march_forward: null ray pointer");
    VGR_REQUIRE(rgb && T && depth && stats, "march_forward: null output pointer");
    const MarchField F{points, offsets, adj, raw, dA, cA, reinterpret_cast<const float4*>(sh), int(sh_deg),
                       int(n_sites)};
    const MarchParams M{float(dt), int(n_bg), float(t_thresh), float(w_thresh)};
    const MarchRays R{o, d, start, near_t, mid_t, far_t, n_rays};
    const MarchOut O{rgb, T, depth, stats, trace, trace_cap};
    if (trace != nullptr)
        hipLaunchKernelGGL(march_forward_kernel<true>, dim3(grid_for(n_rays, kBlock)), dim3(kBlock), 0,
                           as_stream(stream), F, M, R, O);
    else
        hipLaunchKernelGGL(march_forward_kernel<false>, dim3(grid_for(n_rays, kBlock)), dim3(kBlock), 0,
                           as_stream(stream), F, M, R, O);
    return launch_status("march_forward_kernel");
}
