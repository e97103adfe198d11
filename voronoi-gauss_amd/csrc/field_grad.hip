// Backward field operators of the NeRF-style path, gfx950: gradients of density_forward, color_forward and
// conic_forward with respect to the per-site parameters.
//
// Semantics follow csrc/vgf.cu of the reference: scatter_gauss_grad :121-148, density_backward_kernel :179-198,
// color_backward_kernel :284-333, conic_backward_kernel :382-424. With m_k = sum_j y_j^2 / s_j^2, y = R^T (x - p_k):
//   density  dL/draw_k = g rho_k G_k,  dL/dm_k = -g rho_k G_k / 2       (terms with rho_k G_k |g| <= 1e-12 skipped)
//   colour   a_k = softmax(-m / 2)_k, C = sum a_k c_k:  dL/dsh_k = a_k b(d) dL/dC (where SH_k + 1/2 > 0),
//            dL/dm_k = -a_k / 2 (<dL/dC, c_k> - <dL/dC, C>)             (weights a_k < 1e-7 skipped)
//   then dL/dlog_s_k and dL/dq_k from dL/dm_k through the rotation of the normalised quaternion and its tangent
//   projection; conic: A = R diag(1 / (s^2 + floor^2)) R^T, per site, no scatter.
//
// One sample per lane. Per-site gradients are scattered with the hardware fp32 atomics of global memory
// (global_atomic_add_f32 without return, through unsafeAtomicAdd: the gradient buffers are ordinary device
// memory), so their summation order, and the last bits of a sum, vary from run to run. The gradient arrays of the
// density and colour passes are accumulated into: the caller zeroes them.
#include "vgr_abi.h"
#include "vgr_device.h"

namespace vgr {
namespace {

constexpr int kBlock = 256;
constexpr float kMinWeight = 1e-7f;  // normalised colour weights below this get no gradient

struct GradGraph {
    const float* __restrict__ points;  // (N, 3)
    const int* __restrict__ offsets;   // (N + 1)
    const int* __restrict__ adj;       // (M)
    int n_sites;
};

struct GaussIn {
    const float* __restrict__ log_scale;  // (N, 3)
    const float4* __restrict__ quat;      // (N) w x y z, not normalised
};

// Gaussian i seen from (x, y, z): offset v, normalised quaternion qn and the norm it was divided by, rotation R
// (row-major, columns = axes), y = R^T v, inverse variances is2, and m.
struct Frame {
    float v[3], y[3], is2[3], qn[4], qnorm, R[9], m;
};

__device__ __forceinline__ void rotation(float w, float a, float b, float c, float (&R)[9]) {
    R[0] = 1.f - 2.f * (b * b + c * c), R[1] = 2.f * (a * b - w * c), R[2] = 2.f * (a * c + w * b);
    R[3] = 2.f * (a * b + w * c), R[4] = 1.f - 2.f * (a * a + c * c), R[5] = 2.f * (b * c - w * a);
    R[6] = 2.f * (a * c - w * b), R[7] = 2.f * (b * c + w * a), R[8] = 1.f - 2.f * (a * a + b * b);
}

__device__ __forceinline__ void frame_of(const GradGraph& g, const GaussIn& G, int i, float x, float y, float z,
                                         Frame& L) {
    const int64_t i3 = 3 * static_cast<int64_t>(i);
    L.v[0] = x - g.points[i3], L.v[1] = y - g.points[i3 + 1], L.v[2] = z - g.points[i3 + 2];
    const float4 q = G.quat[i];
    L.qnorm = fmaxf(sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w), 1e-12f);
    L.qn[0] = q.x / L.qnorm, L.qn[1] = q.y / L.qnorm, L.qn[2] = q.z / L.qnorm, L.qn[3] = q.w / L.qnorm;
    rotation(L.qn[0], L.qn[1], L.qn[2], L.qn[3], L.R);
    L.m = 0.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        L.y[k] = L.R[k] * L.v[0] + L.R[3 + k] * L.v[1] + L.R[6 + k] * L.v[2];
        const float s = fexp(fminf(fmaxf(G.log_scale[i3 + k], -20.f), 20.f));
        L.is2[k] = 1.f / (s * s);
        L.m += L.y[k] * L.y[k] * L.is2[k];
    }
}

// m alone (the colour pass's first two sweeps), the same arithmetic as frame_of.
__device__ __forceinline__ float maha_of(const GradGraph& g, const GaussIn& G, int i, float x, float y, float z) {
    Frame L;
    frame_of(g, G, i, x, y, z, L);
    return L.m;
}

// dL/dq of R(q / |q|) given dL/dR: the derivative of the rotation in the normalised quaternion, then the tangent
// projection (dq - (dq . qn) qn) / |q| of the normalisation.
__device__ __forceinline__ void quat_grad(const float (&qn)[4], float qnorm, const float (&dR)[9], float (&out)[4]) {
    const float w = qn[0], x = qn[1], y = qn[2], z = qn[3];
    float dq[4];
    dq[0] = 2.f * (-z * dR[1] + y * dR[2] + z * dR[3] - x * dR[5] - y * dR[6] + x * dR[7]);
    dq[1] = 2.f * (y * dR[1] + z * dR[2] + y * dR[3] - 2.f * x * dR[4] - w * dR[5] + z * dR[6] + w * dR[7] -
                   2.f * x * dR[8]);
    dq[2] = 2.f * (-2.f * y * dR[0] + x * dR[1] + w * dR[2] + x * dR[3] + z * dR[5] - w * dR[6] + z * dR[7] -
                   2.f * y * dR[8]);
    dq[3] = 2.f * (-2.f * z * dR[0] - w * dR[1] + x * dR[2] + w * dR[3] - 2.f * z * dR[4] + y * dR[5] + x * dR[6] +
                   y * dR[7]);
    const float proj = dq[0] * w + dq[1] * x + dq[2] * y + dq[3] * z;
#pragma unroll
    for (int k = 0; k < 4; ++k) out[k] = (dq[k] - proj * qn[k]) / qnorm;
}

// Scatters dL/dlog_scale and dL/dquat of Gaussian i given gm = dL/dm.
__device__ __forceinline__ void scatter_gauss(const Frame& L, float gm, int i, float* __restrict__ g_ls,
                                              float* __restrict__ g_quat) {
    float yk[3];
    float* gl = g_ls + 3 * static_cast<int64_t>(i);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        yk[k] = 2.f * gm * L.y[k] * L.is2[k];
        unsafeAtomicAdd(gl + k, -2.f * gm * L.y[k] * L.y[k] * L.is2[k]);
    }
    float dR[9];  // dL/dR_ab = v_a dL/dy_b
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int b = 0; b < 3; ++b) dR[3 * a + b] = L.v[a] * yk[b];
    float gq[4];
    quat_grad(L.qn, L.qnorm, dR, gq);
    float* gqp = g_quat + 4 * static_cast<int64_t>(i);
#pragma unroll
    for (int k = 0; k < 4; ++k) unsafeAtomicAdd(gqp + k, gq[k]);
}

__global__ void __launch_bounds__(kBlock)
    density_backward_kernel(GradGraph g, const float* __restrict__ raw, GaussIn G, const float* __restrict__ x,
                            const int* __restrict__ site, int64_t m, const float* __restrict__ grad_sigma,
                            float* __restrict__ g_raw, float* __restrict__ g_ls, float* __restrict__ g_quat) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= m) return;
    const float gs = grad_sigma[t];
    const int i = site[t];
    if (gs == 0.f || i < 0 || i >= g.n_sites) return;  // an unresolved sample has sigma 0 and no gradient
    const float qx = x[3 * t], qy = x[3 * t + 1], qz = x[3 * t + 2];
    const int e0 = g.offsets[i], e1 = g.offsets[i + 1];
    for (int e = e0 - 1; e < e1; ++e) {
        const int k = e < e0 ? i : g.adj[e];
        Frame L;
        frame_of(g, G, k, qx, qy, qz, L);
        const float c = fexp(fminf(raw[k], 30.f) - 0.5f * L.m);  // rho_k G_k
        if (c * fabsf(gs) > 1e-12f) {
            unsafeAtomicAdd(g_raw + k, gs * c);
            scatter_gauss(L, -0.5f * gs * c, k, g_ls, g_quat);
        }
    }
}

template <int DEG>
__global__ void __launch_bounds__(kBlock)
    color_backward_kernel(GradGraph g, GaussIn H, const float4* __restrict__ sh, const float* __restrict__ x,
                          const float* __restrict__ dirs, const int* __restrict__ site, int64_t m,
                          const float* __restrict__ rgb, const float* __restrict__ grad_rgb, float* __restrict__ g_ls,
                          float* __restrict__ g_quat, float* __restrict__ g_sh) {
    constexpr int nb = (DEG + 1) * (DEG + 1);
    constexpr int NV = sh_vec4_f32(DEG);
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= m) return;
    const float gr = grad_rgb[3 * t], gg = grad_rgb[3 * t + 1], gb = grad_rgb[3 * t + 2];
    const int i = site[t];
    if ((gr == 0.f && gg == 0.f && gb == 0.f) || i < 0 || i >= g.n_sites) return;
    const float qx = x[3 * t], qy = x[3 * t + 1], qz = x[3 * t + 2];
    const int e0 = g.offsets[i], e1 = g.offsets[i + 1];
    float mmin = kInf;
    for (int e = e0 - 1; e < e1; ++e) mmin = fminf(mmin, maha_of(g, H, e < e0 ? i : g.adj[e], qx, qy, qz));
    float A = 0.f;
    for (int e = e0 - 1; e < e1; ++e) A += fexp(-0.5f * (maha_of(g, H, e < e0 ? i : g.adj[e], qx, qy, qz) - mmin));
    const float inv_a = 1.f / A;
    const float gCC = gr * rgb[3 * t] + gg * rgb[3 * t + 1] + gb * rgb[3 * t + 2];
    float dx = dirs[3 * t], dy = dirs[3 * t + 1], dz = dirs[3 * t + 2];
    const float inv = rsqrtf(fmaxf(dx * dx + dy * dy + dz * dz, 1e-20f));
    dx *= inv, dy *= inv, dz *= inv;
    float b[16];
    sh_basis(dx, dy, dz, DEG, b);
    for (int e = e0 - 1; e < e1; ++e) {
        const int k = e < e0 ? i : g.adj[e];
        Frame L;
        frame_of(g, H, k, qx, qy, qz, L);
        const float a = fexp(-0.5f * (L.m - mmin)) * inv_a;
        if (a < kMinWeight) continue;
        // c_k = SH_k(d) + 1/2 over the coefficients of degree <= DEG (storage order: coefficient j, channel c at
        // 3 j + c)
        const float4* s = sh + 12 * static_cast<int64_t>(k);
        float c[3] = {0.5f, 0.5f, 0.5f};
#pragma unroll
        for (int q = 0; q < NV; ++q) {
            const float4 f = s[q];
            const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = 4 * q + u;
                if (j / 3 < nb) c[j % 3] += b[j / 3] * fv[u];
            }
        }
        const float dc[3] = {c[0] > 0.f ? a * gr : 0.f, c[1] > 0.f ? a * gg : 0.f, c[2] > 0.f ? a * gb : 0.f};
        float* gsh = g_sh + 48 * static_cast<int64_t>(k);
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) {
            if (dc[ch] == 0.f) continue;
#pragma unroll
            for (int j = 0; j < nb; ++j) unsafeAtomicAdd(gsh + 3 * j + ch, b[j] * dc[ch]);
        }
        const float ga = gr * fmaxf(c[0], 0.f) + gg * fmaxf(c[1], 0.f) + gb * fmaxf(c[2], 0.f);
        const float gm = -0.5f * a * (ga - gCC);
        if (gm != 0.f) scatter_gauss(L, gm, k, g_ls, g_quat);
    }
}

__global__ void __launch_bounds__(kBlock)
    conic_backward_kernel(const float* __restrict__ log_scale, const float4* __restrict__ quat, int64_t n,
                          float floor2, const float* __restrict__ gA, float* __restrict__ g_ls,
                          float* __restrict__ g_quat) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    const float4 q = quat[i];
    const float qnorm = fmaxf(sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w), 1e-12f);
    const float qn[4] = {q.x / qnorm, q.y / qnorm, q.z / qnorm, q.w / qnorm};
    float R[9];
    rotation(qn[0], qn[1], qn[2], qn[3], R);
    float iv[3], s2[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        s2[k] = fexp(2.f * fminf(fmaxf(log_scale[3 * i + k], -20.f), 20.f));
        iv[k] = 1.f / (s2[k] + floor2);
    }
    // the off-diagonal entries of A stand for A_ab and A_ba: dL/dA is symmetric with half of them off the diagonal
    const float* ga = gA + 6 * i;
    const float G[9] = {ga[0],        0.5f * ga[1], 0.5f * ga[2], 0.5f * ga[1], ga[3],
                        0.5f * ga[4], 0.5f * ga[2], 0.5f * ga[4], ga[5]};
    float GR[9];
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int k = 0; k < 3; ++k) GR[3 * r + k] = G[3 * r] * R[k] + G[3 * r + 1] * R[3 + k] + G[3 * r + 2] * R[6 + k];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const float g_iv = R[k] * GR[k] + R[3 + k] * GR[3 + k] + R[6 + k] * GR[6 + k];  // (R^T G R)_kk
        g_ls[3 * i + k] = g_iv * (-2.f * s2[k] * iv[k] * iv[k]);
    }
    float dR[9];  // dL/dR = 2 G R diag(iv)
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int k = 0; k < 3; ++k) dR[3 * r + k] = 2.f * GR[3 * r + k] * iv[k];
    float gq[4];
    quat_grad(qn, qnorm, dR, gq);
#pragma unroll
    for (int k = 0; k < 4; ++k) g_quat[4 * i + k] = gq[k];
}

int check_grad_graph(const char* op, const float* points, int64_t n_sites, const int32_t* offsets,
                     const int32_t* adj, int64_t n_adj) {
    VGR_REQUIRE(n_sites > 0 && n_sites <= INT_MAX, "%s: n_sites must be in [1, 2^31)", op);
    VGR_REQUIRE(n_adj >= 0 && n_adj <= INT_MAX, "%s: n_adj must be in [0, 2^31)", op);
    VGR_REQUIRE(points && offsets && (adj || n_adj == 0), "%s: null graph pointer", op);
    return VGR_OK;
}

}  // namespace
}  // namespace vgr

extern "C" int vgr_density_backward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                                    int64_t n_adj, const float* raw, const float* log_scale, const float* quat,
                                    const float* x, const int32_t* site, int64_t m, const float* grad_sigma,
                                    float* g_raw, float* g_ls, float* g_quat, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(m >= 0, "density_backward: m must be >= 0");
    if (m == 0) return VGR_OK;
    if (int rc = check_grad_graph("density_backward", points, n_sites, offsets, adj, n_adj)) return rc;
    VGR_REQUIRE(raw && log_scale && quat && x && site && grad_sigma && g_raw && g_ls && g_quat,
                "density_backward: null pointer");
    hipLaunchKernelGGL(density_backward_kernel, dim3(grid_for(m, kBlock)), dim3(kBlock), 0, as_stream(stream),
                       GradGraph{points, offsets, adj, int(n_sites)},
                       raw, GaussIn{log_scale, reinterpret_cast<const float4*>(quat)}, x, site, m, grad_sigma, g_raw,
                       g_ls, g_quat);
    return launch_status("density_backward_kernel");
}

extern "C" int vgr_color_backward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                                  int64_t n_adj, const float* log_scale, const float* quat, const float* sh,
                                  int64_t sh_deg, const float* x, const float* dirs, const int32_t* site, int64_t m,
                                  const float* rgb, const float* grad_rgb, float* g_ls, float* g_quat, float* g_sh,
                                  void* stream) {
    using namespace vgr;
    VGR_REQUIRE(m >= 0, "color_backward: m must be >= 0");
    VGR_REQUIRE(sh_deg >= 0 && sh_deg <= 3, "sh_deg must be in [0, 3] (got %lld)", static_cast<long long>(sh_deg));
    if (m == 0) return VGR_OK;
    if (int rc = check_grad_graph("color_backward", points, n_sites, offsets, adj, n_adj)) return rc;
    VGR_REQUIRE(log_scale && quat && sh && x && dirs && site && rgb && grad_rgb && g_ls && g_quat && g_sh,
                "color_backward: null pointer");
    const GradGraph g{points, offsets, adj, int(n_sites)};
    const GaussIn H{log_scale, reinterpret_cast<const float4*>(quat)};
    const float4* s4 = reinterpret_cast<const float4*>(sh);
    const dim3 grid(grid_for(m, kBlock)), block(kBlock);
    const hipStream_t st = as_stream(stream);
    switch (sh_deg) {
        case 0:
            hipLaunchKernelGGL(color_backward_kernel<0>, grid, block, 0, st, g, H, s4, x, dirs, site, m, rgb,
                               grad_rgb, g_ls, g_quat, g_sh);
            break;
        case 1:
            hipLaunchKernelGGL(color_backward_kernel<1>, grid, block, 0, st, g, H, s4, x, dirs, site, m, rgb,
                               grad_rgb, g_ls, g_quat, g_sh);
            break;
        case 2:
            hipLaunchKernelGGL(color_backward_kernel<2>, grid, block, 0, st, g, H, s4, x, dirs, site, m, rgb,
                               grad_rgb, g_ls, g_quat, g_sh);
            break;
        default:
            hipLaunchKernelGGL(color_backward_kernel<3>, grid, block, 0, st, g, H, s4, x, dirs, site, m, rgb,
                               grad_rgb, g_ls, g_quat, g_sh);
            break;
    }
    return launch_status("color_backward_kernel");
}

extern "C" int vgr_conic_backward(const float* log_scale, const float* quat, int64_t n, double floor, const float* gA,
                                  float* g_ls, float* g_quat, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(n >= 0, "conic_backward: n must be >= 0");
    if (n == 0) return VGR_OK;
    VGR_REQUIRE(log_scale && quat && gA && g_ls && g_quat, "conic_backward: null pointer");
    hipLaunchKernelGGL(conic_backward_kernel, dim3(grid_for(n, kBlock)), dim3(kBlock), 0, as_stream(stream),
                       log_scale, reinterpret_cast<const float4*>(quat), n, static_cast<float>(floor * floor), gA,
                       g_ls, g_quat);
    return launch_status("conic_backward_kernel");
}
