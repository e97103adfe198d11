// Backward field operators of the NeRF-style path, gfx950: gradients of density_forward, color_forward and
// conic_forward with respect to the per-site parameters.
//
// Semantics follow csrc/vgf.cu of the reference: scatter_gauss_grad :121-148 (here add_gauss_grad, with dL/dq in
// the outer-product form derived at quat_grad_of), density_backward_kernel :179-198,
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
//
// Scattered, the colour pass issues up to 55 atomics per (sample, neighbour) pair (48 of them SH coefficients,
// 86 % of its time) and the density pass 8. Given a workspace, both gather instead (measured on config 3 training
// batches: colour 4.7 -> 1.1 ms for 4096 rays; density 1.07 -> 2.6 ms, slower, since its lane per site runs as long
// as the busiest site of its wave, so the host wrapper gathers colour only): the samples are counting-sorted
// by site into packed records, and one lane per site k walks the samples of its own and its Delaunay neighbours'
// cells (k is in the neighbourhood of a sample of cell i exactly when i is k or a neighbour of k), accumulates its
// gradients in registers and adds them once, without atomics. The log-scale and quaternion gradients are linear in
// the per-site sums S_j = sum gm y_j^2 and G_ab = sum gm v_a y_b (the rotation, variances and quaternion are the
// site's), so the quaternion derivative is applied once per site.
#include "vgr_abi.h"
#include "vgr_device.h"
#include "vgr_scan.h"

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

// A site's Gaussian as the gradients need it, built once per (site, use): the unit quaternion (w, u) and the norm
// |q| it was divided by, the axes of the Gaussian (the columns of R(q / |q|)), the inverse variances 1 / s_j^2 and the
// position.
struct SiteGauss {
    float w, u[3], qnorm;
    float axis[3][3];  // axis[j] = column j of R
    float is2[3];
    float p[3];
};

__device__ __forceinline__ void unit_quat(const float4& q, float& w, float (&u)[3], float& qnorm) {
    qnorm = fmaxf(sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w), 1e-12f);
    w = q.x / qnorm, u[0] = q.y / qnorm, u[1] = q.z / qnorm, u[2] = q.w / qnorm;
}

// Columns of the rotation of the unit quaternion (w, u): the images of the coordinate axes.
__device__ __forceinline__ void quat_axes(float w, const float (&u)[3], float (&axis)[3][3]) {
    const float xx = u[0] * u[0], yy = u[1] * u[1], zz = u[2] * u[2];
    const float xy = u[0] * u[1], xz = u[0] * u[2], yz = u[1] * u[2];
    const float wx = w * u[0], wy = w * u[1], wz = w * u[2];
    axis[0][0] = 1.f - 2.f * (yy + zz), axis[0][1] = 2.f * (xy + wz), axis[0][2] = 2.f * (xz - wy);
    axis[1][0] = 2.f * (xy - wz), axis[1][1] = 1.f - 2.f * (xx + zz), axis[1][2] = 2.f * (yz + wx);
    axis[2][0] = 2.f * (xz + wy), axis[2][1] = 2.f * (yz - wx), axis[2][2] = 1.f - 2.f * (xx + yy);
}

__device__ __forceinline__ SiteGauss site_gauss(const GradGraph& g, const GaussIn& G, int i) {
    SiteGauss S;
    unit_quat(G.quat[i], S.w, S.u, S.qnorm);
    quat_axes(S.w, S.u, S.axis);
    const int64_t i3 = 3 * static_cast<int64_t>(i);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const float s = fexp(fminf(fmaxf(G.log_scale[i3 + j], -20.f), 20.f));
        S.is2[j] = 1.f / (s * s);
        S.p[j] = g.points[i3 + j];
    }
    return S;
}

// Offset v = x - p, local coordinates y_j = axis_j . v and the Mahalanobis distance m = sum_j y_j^2 / s_j^2.
__device__ __forceinline__ float site_local(const SiteGauss& S, float x, float y, float z, float (&v)[3],
                                            float (&yl)[3]) {
    v[0] = x - S.p[0], v[1] = y - S.p[1], v[2] = z - S.p[2];
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        yl[j] = S.axis[j][0] * v[0] + S.axis[j][1] * v[1] + S.axis[j][2] * v[2];
        m += yl[j] * yl[j] * S.is2[j];
    }
    return m;
}

// m of site i at x (the colour gradient's first sweeps), site_local's arithmetic.
__device__ __forceinline__ float site_m(const GradGraph& g, const GaussIn& G, int i, float x, float y, float z) {
    const SiteGauss S = site_gauss(g, G, i);
    float v[3], yl[3];
    return site_local(S, x, y, z, v, yl);
}

// dL/dq for a loss that depends on q through R(q / |q|), given M = dL/dR (row-major, M[3a + b] = dL/dR_ab). With
// R^T v = v - 2 w (u x v) + 2 u (u . v) - 2 v |u|^2 (Rodrigues' form of the rotation of the unit quaternion (w, u),
// treated as a polynomial in (w, u)), and ax(M) = (M_12 - M_21, M_20 - M_02, M_01 - M_10):
//   dL/dw = -2 u . ax(M),    dL/du = -2 w ax(M) + 2 (M u + M^T u) - 4 tr(M) u,
// then the tangent projection of the normalisation: (d - (d . q^) q^) / |q|.
__device__ __forceinline__ void quat_grad_of(float w, const float (&u)[3], float qnorm, const float (&M)[9],
                                             float (&out)[4]) {
    const float ax[3] = {M[5] - M[7], M[6] - M[2], M[1] - M[3]};
    const float tr = M[0] + M[4] + M[8];
    float d[4];
    d[0] = -2.f * (u[0] * ax[0] + u[1] * ax[1] + u[2] * ax[2]);
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const float Mu = M[3 * a] * u[0] + M[3 * a + 1] * u[1] + M[3 * a + 2] * u[2];
        const float MTu = M[a] * u[0] + M[3 + a] * u[1] + M[6 + a] * u[2];
        d[1 + a] = -2.f * w * ax[a] + 2.f * (Mu + MTu) - 4.f * tr * u[a];
    }
    const float radial = d[0] * w + d[1] * u[0] + d[2] * u[1] + d[3] * u[2];
    out[0] = (d[0] - radial * w) / qnorm;
#pragma unroll
    for (int a = 0; a < 3; ++a) out[1 + a] = (d[1 + a] - radial * u[a]) / qnorm;
}

// Adds the log-scale and quaternion gradients of site k for dL/dm = gm at offset v (local coordinates yl):
// dm/dlog_s_j = -2 y_j^2 / s_j^2, and dL/dR_ab = v_a dL/dy_b with dL/dy_b = 2 gm y_b / s_b^2.
__device__ __forceinline__ void add_gauss_grad(const SiteGauss& S, float gm, const float (&v)[3],
                                               const float (&yl)[3], int k, float* __restrict__ g_ls,
                                               float* __restrict__ g_quat) {
    float gy[3], M[9];
    float* gl = g_ls + 3 * static_cast<int64_t>(k);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        gy[j] = 2.f * gm * yl[j] * S.is2[j];
        unsafeAtomicAdd(gl + j, -gy[j] * yl[j]);
    }
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int b = 0; b < 3; ++b) M[3 * a + b] = v[a] * gy[b];
    float gq[4];
    quat_grad_of(S.w, S.u, S.qnorm, M, gq);
    float* gqp = g_quat + 4 * static_cast<int64_t>(k);
#pragma unroll
    for (int j = 0; j < 4; ++j) unsafeAtomicAdd(gqp + j, gq[j]);
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
        const SiteGauss S = site_gauss(g, G, k);
        float v[3], yl[3];
        const float c = fexp(fminf(raw[k], 30.f) - 0.5f * site_local(S, qx, qy, qz, v, yl));  // rho_k G_k
        if (c * fabsf(gs) > 1e-12f) {
            unsafeAtomicAdd(g_raw + k, gs * c);
            add_gauss_grad(S, -0.5f * gs * c, v, yl, k, g_ls, g_quat);
        }
    }
}

// Per-sample record of the SH gather: x, the unit direction, dL/dC, mmin and 1 / A of the sample's blend.
struct SampleRec {
    float4 a;  // x (3), mmin
    float4 b;  // unit direction (3), 1 / A
    float4 c;  // dL/dC (3), <dL/dC, C>
};

// Per-site sums of the log-scale and quaternion gradients (see the header): S_j = sum gm y_j^2,
// G_ab = sum gm v_a y_b.
struct GaussSums {
    float S[3], G[9];
};

__device__ __forceinline__ void sums_init(GaussSums& A) {
#pragma unroll
    for (int j = 0; j < 3; ++j) A.S[j] = 0.f;
#pragma unroll
    for (int j = 0; j < 9; ++j) A.G[j] = 0.f;
}

__device__ __forceinline__ void sums_add(GaussSums& A, float gm, const float (&v)[3], const float (&y)[3]) {
#pragma unroll
    for (int j = 0; j < 3; ++j) A.S[j] += gm * y[j] * y[j];
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int b = 0; b < 3; ++b) A.G[3 * a + b] += gm * v[a] * y[b];
}

// Adds site k's log-scale and quaternion gradients from its sums (F: the site's frame).
__device__ __forceinline__ void sums_write(const GaussSums& A, const SiteGauss& F, int64_t k,
                                           float* __restrict__ g_ls, float* __restrict__ g_quat) {
    float M[9];  // dL/dR
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int b = 0; b < 3; ++b) M[3 * a + b] = 2.f * F.is2[b] * A.G[3 * a + b];
    float gq[4];
    quat_grad_of(F.w, F.u, F.qnorm, M, gq);
#pragma unroll
    for (int j = 0; j < 3; ++j) g_ls[3 * k + j] += -2.f * F.is2[j] * A.S[j];
#pragma unroll
    for (int j = 0; j < 4; ++j) g_quat[4 * k + j] += gq[j];
}

// SH_k(d) + 1/2 over the coefficients of degree <= DEG (storage order: coefficient j, channel c at 3 j + c).
template <int DEG>
__device__ __forceinline__ void sh_colour(const float4* __restrict__ s, const float (&b)[16], float (&c)[3]) {
    constexpr int nb = (DEG + 1) * (DEG + 1);
    c[0] = c[1] = c[2] = 0.5f;
#pragma unroll
    for (int q = 0; q < sh_vec4_f32(DEG); ++q) {
        const float4 f = s[q];
        const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = 4 * q + u;
            if (j / 3 < nb) c[j % 3] += b[j / 3] * fv[u];
        }
    }
}

// GATHER: the SH gradient is left to colour_sh_gather_kernel; the sample's blend (mmin, 1 / A) is written to
// rec_of[t] instead (the sorted position of the sample, or -1 when it contributes nothing).
template <int DEG, bool GATHER>
__global__ void __launch_bounds__(kBlock)
    color_backward_kernel(GradGraph g, GaussIn H, const float4* __restrict__ sh, const float* __restrict__ x,
                          const float* __restrict__ dirs, const int* __restrict__ site, int64_t m,
                          const float* __restrict__ rgb, const float* __restrict__ grad_rgb, float* __restrict__ g_ls,
                          float* __restrict__ g_quat, float* __restrict__ g_sh, const int* __restrict__ slot,
                          SampleRec* __restrict__ recs) {
    constexpr int nb = (DEG + 1) * (DEG + 1);
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= m) return;
    const float gr = grad_rgb[3 * t], gg = grad_rgb[3 * t + 1], gb = grad_rgb[3 * t + 2];
    const int i = site[t];
    if ((gr == 0.f && gg == 0.f && gb == 0.f) || i < 0 || i >= g.n_sites) return;
    const float qx = x[3 * t], qy = x[3 * t + 1], qz = x[3 * t + 2];
    const int e0 = g.offsets[i], e1 = g.offsets[i + 1];
    float mmin = kInf;
    for (int e = e0 - 1; e < e1; ++e) mmin = fminf(mmin, site_m(g, H, e < e0 ? i : g.adj[e], qx, qy, qz));
    float A = 0.f;
    for (int e = e0 - 1; e < e1; ++e) A += fexp(-0.5f * (site_m(g, H, e < e0 ? i : g.adj[e], qx, qy, qz) - mmin));
    const float inv_a = 1.f / A;
    const float gCC = gr * rgb[3 * t] + gg * rgb[3 * t + 1] + gb * rgb[3 * t + 2];
    float dx = dirs[3 * t], dy = dirs[3 * t + 1], dz = dirs[3 * t + 2];
    const float inv = rsqrtf(fmaxf(dx * dx + dy * dy + dz * dz, 1e-20f));
    dx *= inv, dy *= inv, dz *= inv;
    float b[16];
    sh_basis(dx, dy, dz, DEG, b);
    if constexpr (GATHER) {  // the per-site gather does the rest
        SampleRec r;
        r.a = make_float4(qx, qy, qz, mmin), r.b = make_float4(dx, dy, dz, inv_a), r.c = make_float4(gr, gg, gb, gCC);
        recs[slot[t]] = r;
        return;
    }
    for (int e = e0 - 1; e < e1; ++e) {
        const int k = e < e0 ? i : g.adj[e];
        const SiteGauss S = site_gauss(g, H, k);
        float v[3], yl[3];
        const float a = fexp(-0.5f * (site_local(S, qx, qy, qz, v, yl) - mmin)) * inv_a;
        if (a < kMinWeight) continue;
        float c[3];
        sh_colour<DEG>(sh + 12 * static_cast<int64_t>(k), b, c);
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
        if (gm != 0.f) add_gauss_grad(S, gm, v, yl, k, g_ls, g_quat);
    }
}

// The samples that contribute (a valid site and a non-zero dL/dC) are counted per site; slot[t] = -1 for the
// others.
// A sample contributes when its site is valid and its upstream gradient (W floats) is not all zero.
template <int W>
__device__ __forceinline__ bool contributes(const GradGraph& g, const int* __restrict__ site,
                                            const float* __restrict__ grad, int64_t t) {
    const int i = site[t];
    if (i < 0 || i >= g.n_sites) return false;
    bool nz = false;
#pragma unroll
    for (int u = 0; u < W; ++u) nz = nz || grad[W * t + u] != 0.f;
    return nz;
}

template <int W>
__global__ void __launch_bounds__(kBlock)
    sample_count_kernel(GradGraph g, const int* __restrict__ site, const float* __restrict__ grad, int64_t m,
                        int* __restrict__ count) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= m) return;
    if (contributes<W>(g, site, grad, t)) atomicAdd(count + site[t], 1);
}

__global__ void __launch_bounds__(kBlock) fill_zero_kernel(int* __restrict__ p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i < n) p[i] = 0;
}

// Every contributing sample takes the next record slot of its site (the order within a site is arbitrary: the
// gather sums over all of them).
template <int W>
__global__ void __launch_bounds__(kBlock)
    sample_slot_kernel(GradGraph g, const int* __restrict__ site, const float* __restrict__ grad, int64_t m,
                       int* __restrict__ cursor, int* __restrict__ slot) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= m) return;
    slot[t] = contributes<W>(g, site, grad, t) ? atomicAdd(cursor + site[t], 1) : -1;
}

// Density records: the sample's position and dL/dsigma, at the sample's slot.
__global__ void __launch_bounds__(kBlock)
    density_record_kernel(const float* __restrict__ x, const float* __restrict__ grad_sigma, int64_t m,
                          const int* __restrict__ slot, float4* __restrict__ recs) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= m || slot[t] < 0) return;
    recs[slot[t]] = make_float4(x[3 * t], x[3 * t + 1], x[3 * t + 2], grad_sigma[t]);
}

// Density gradients of site k gathered over the samples of the cells {k} U adj(k): the same terms as
// density_backward_kernel (rho_k G_k |dL/dsigma| <= 1e-12 skipped), summed per site.
__global__ void __launch_bounds__(kBlock)
    density_gather_kernel(GradGraph g, const float* __restrict__ raw, GaussIn G, const int* __restrict__ start,
                          const float4* __restrict__ recs, float* __restrict__ g_raw, float* __restrict__ g_ls,
                          float* __restrict__ g_quat) {
    const int64_t kk = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (kk >= g.n_sites) return;
    const int k = static_cast<int>(kk);
    const SiteGauss F = site_gauss(g, G, k);
    const float raw_c = fminf(raw[k], 30.f);
    GaussSums A;
    sums_init(A);
    float acc_raw = 0.f;
    bool any = false;
    const int e0 = g.offsets[k], e1 = g.offsets[k + 1];
    for (int e = e0 - 1; e < e1; ++e) {
        const int i = e < e0 ? k : g.adj[e];
        const int r1 = start[i + 1];
        for (int r = start[i]; r < r1; ++r) {
            const float4 rec = recs[r];
            float v[3], y[3];
            const float m_k = site_local(F, rec.x, rec.y, rec.z, v, y);
            const float c = fexp(raw_c - 0.5f * m_k);  // rho_k G_k
            if (c * fabsf(rec.w) > 1e-12f) {
                acc_raw += rec.w * c;
                sums_add(A, -0.5f * rec.w * c, v, y);
                any = true;
            }
        }
    }
    if (!any) return;
    g_raw[kk] += acc_raw;
    sums_write(A, F, kk, g_ls, g_quat);
}

// Colour gradients of site k gathered over the samples t of the cells {k} U adj(k): dL/dsh = sum a_tk b(d_t)
// (dL/dC_t on the channels where SH_k(d_t) + 1/2 > 0) and dL/dm_tk = -a_tk / 2 (<dL/dC_t, c_k> - <dL/dC_t, C_t>),
// with a_tk = exp(-(m_tk - mmin_t) / 2) / A_t from the sample's record; weights below 1e-7 are skipped, as in the
// scatter.
template <int DEG>
__global__ void __launch_bounds__(kBlock)
    colour_gather_kernel(GradGraph g, GaussIn H, const float4* __restrict__ sh, const int* __restrict__ start,
                         const SampleRec* __restrict__ recs, float* __restrict__ g_ls, float* __restrict__ g_quat,
                         float* __restrict__ g_sh) {
    constexpr int nb = (DEG + 1) * (DEG + 1);
    const int64_t kk = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (kk >= g.n_sites) return;
    const int k = static_cast<int>(kk);
    const int e0 = g.offsets[k], e1 = g.offsets[k + 1];
    float acc[nb][3];
#pragma unroll
    for (int j = 0; j < nb; ++j) acc[j][0] = acc[j][1] = acc[j][2] = 0.f;
    bool any = false;
    const float4* sk = sh + 12 * kk;
    const SiteGauss F = site_gauss(g, H, k);
    GaussSums A;
    sums_init(A);
    for (int e = e0 - 1; e < e1; ++e) {
        const int i = e < e0 ? k : g.adj[e];
        const int r0 = start[i], r1 = start[i + 1];
        for (int r = r0; r < r1; ++r) {
            const SampleRec rec = recs[r];
            float v[3], y[3];
            const float m_k = site_local(F, rec.a.x, rec.a.y, rec.a.z, v, y);
            const float a = fexp(-0.5f * (m_k - rec.a.w)) * rec.b.w;
            if (a < kMinWeight) continue;
            float b[16];
            sh_basis(rec.b.x, rec.b.y, rec.b.z, DEG, b);
            float c[3];
            sh_colour<DEG>(sk, b, c);
            const float dc[3] = {c[0] > 0.f ? a * rec.c.x : 0.f, c[1] > 0.f ? a * rec.c.y : 0.f,
                                 c[2] > 0.f ? a * rec.c.z : 0.f};
#pragma unroll
            for (int j = 0; j < nb; ++j)
#pragma unroll
                for (int ch = 0; ch < 3; ++ch) acc[j][ch] += b[j] * dc[ch];
            const float ga = rec.c.x * fmaxf(c[0], 0.f) + rec.c.y * fmaxf(c[1], 0.f) + rec.c.z * fmaxf(c[2], 0.f);
            sums_add(A, -0.5f * a * (ga - rec.c.w), v, y);
            any = true;
        }
    }
    if (!any) return;
    float* gsh = g_sh + 48 * kk;
#pragma unroll
    for (int j = 0; j < nb; ++j)
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) gsh[3 * j + ch] += acc[j][ch];
    sums_write(A, F, kk, g_ls, g_quat);
}

// Workspace of the gathers for n sites and m samples (sections 256-byte aligned): int count[n + 1] (the slot
// cursor after the scan), int start[n + 1], int tile_sum[tiles + 1], int slot[m], records[m] (SampleRec for colour,
// float4 for density).
constexpr int64_t align256b(int64_t b) { return (b + 255) / 256 * 256; }

int64_t gather_bytes(int64_t n, int64_t m) {
    return 2 * align256b(4 * (n + 1)) + align256b(4 * (scan_tiles_of(n) + 1)) + align256b(4 * m) +
           align256b(static_cast<int64_t>(sizeof(SampleRec)) * m);
}

__global__ void __launch_bounds__(kBlock)
    conic_backward_kernel(const float* __restrict__ log_scale, const float4* __restrict__ quat, int64_t n,
                          float floor2, const float* __restrict__ gA, float* __restrict__ g_ls,
                          float* __restrict__ g_quat) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    // A = sum_j iv_j a_j a_j^T over the axes a_j (columns of R), iv_j = 1 / (s_j^2 + floor^2); dL/dA is symmetric,
    // its off-diagonal storage entries standing for both A_ab and A_ba
    float w, u[3], qnorm, axis[3][3];
    unit_quat(quat[i], w, u, qnorm);
    quat_axes(w, u, axis);
    const float* ga = gA + 6 * i;
    const float G[3][3] = {{ga[0], 0.5f * ga[1], 0.5f * ga[2]},
                           {0.5f * ga[1], ga[3], 0.5f * ga[4]},
                           {0.5f * ga[2], 0.5f * ga[4], ga[5]}};
    float M[9];  // dL/dR: column j is 2 iv_j G a_j
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const float s2 = fexp(2.f * fminf(fmaxf(log_scale[3 * i + j], -20.f), 20.f));
        const float iv = 1.f / (s2 + floor2);
        float Ga[3];
#pragma unroll
        for (int a = 0; a < 3; ++a) Ga[a] = G[a][0] * axis[j][0] + G[a][1] * axis[j][1] + G[a][2] * axis[j][2];
        const float aGa = axis[j][0] * Ga[0] + axis[j][1] * Ga[1] + axis[j][2] * Ga[2];  // dL/div_j
        g_ls[3 * i + j] = aGa * (-2.f * s2 * iv * iv);                                   // div_j/dlog_s_j
#pragma unroll
        for (int a = 0; a < 3; ++a) M[3 * a + j] = 2.f * iv * Ga[a];
    }
    float gq[4];
    quat_grad_of(w, u, qnorm, M, gq);
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

namespace vgr {
namespace {

// Counting sort of the contributing samples by site: start[0 .. n] = first slot of each site's samples,
// slot[t] = the sample's slot (-1 when it contributes nothing).
template <int W>
void sort_samples(const GradGraph& g, const int32_t* site, const float* grad, int64_t m, int* count, int* start,
                  int* tile_sum, int* slot, hipStream_t st) {
    const int64_t n = g.n_sites;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(n, kBlock)), dim3(kBlock), 0, st, count, n);
    hipLaunchKernelGGL(sample_count_kernel<W>, dim3(grid_for(m, kBlock)), dim3(kBlock), 0, st, g, site, grad, m, count);
    exclusive_scan(count, n, start, count, tile_sum, st);  // count becomes the slot cursor
    hipLaunchKernelGGL(sample_slot_kernel<W>, dim3(grid_for(m, kBlock)), dim3(kBlock), 0, st, g, site, grad, m, count,
                       slot);
}

// The sections of a gather workspace.
struct GatherWork {
    int *count, *start, *tile_sum, *slot;
    void* recs;
};

GatherWork gather_work(void* work, int64_t n, int64_t m) {
    char* w = static_cast<char*>(work);
    GatherWork W;
    W.count = reinterpret_cast<int*>(w);
    w += align256b(4 * (n + 1));
    W.start = reinterpret_cast<int*>(w);
    w += align256b(4 * (n + 1));
    W.tile_sum = reinterpret_cast<int*>(w);
    w += align256b(4 * (scan_tiles_of(n) + 1));
    W.slot = reinterpret_cast<int*>(w);
    w += align256b(4 * m);
    W.recs = w;
    return W;
}

template <int DEG>
int color_backward_launch(const GradGraph& g, const GaussIn& H, const float4* sh, const float* x, const float* dirs,
                          const int32_t* site, int64_t m, const float* rgb, const float* grad_rgb, float* g_ls,
                          float* g_quat, float* g_sh, void* work, hipStream_t st) {
    const dim3 grid(grid_for(m, kBlock)), block(kBlock);
    if (work == nullptr) {
        hipLaunchKernelGGL((color_backward_kernel<DEG, false>), grid, block, 0, st, g, H, sh, x, dirs, site, m, rgb,
                           grad_rgb, g_ls, g_quat, g_sh, nullptr, nullptr);
        return launch_status("color_backward_kernel");
    }
    const int64_t n = g.n_sites;
    const GatherWork W = gather_work(work, n, m);
    int *start = W.start, *slot = W.slot;
    SampleRec* recs = static_cast<SampleRec*>(W.recs);
    sort_samples<3>(g, site, grad_rgb, m, W.count, start, W.tile_sum, slot, st);
    hipLaunchKernelGGL((color_backward_kernel<DEG, true>), grid, block, 0, st, g, H, sh, x, dirs, site, m, rgb,
                       grad_rgb, g_ls, g_quat, g_sh, slot, recs);
    hipLaunchKernelGGL(colour_gather_kernel<DEG>, dim3(grid_for(n, kBlock)), block, 0, st, g, H, sh, start, recs,
                       g_ls, g_quat, g_sh);
    return launch_status("color_backward_kernel / colour_gather_kernel");
}

}  // namespace
}  // namespace vgr

extern "C" int64_t vgr_density_backward_work_size(int64_t n_sites, int64_t m) {
    return n_sites > 0 && m >= 0 ? vgr::gather_bytes(n_sites, m) : 0;
}

extern "C" int vgr_density_backward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                                    int64_t n_adj, const float* raw, const float* log_scale, const float* quat,
                                    const float* x, const int32_t* site, int64_t m, const float* grad_sigma,
                                    float* g_raw, float* g_ls, float* g_quat, void* work, int64_t work_bytes,
                                    void* stream) {
    using namespace vgr;
    VGR_REQUIRE(m >= 0, "density_backward: m must be >= 0");
    if (m == 0) return VGR_OK;
    if (int rc = check_grad_graph("density_backward", points, n_sites, offsets, adj, n_adj)) return rc;
    VGR_REQUIRE(raw && log_scale && quat && x && site && grad_sigma && g_raw && g_ls && g_quat,
                "density_backward: null pointer");
    VGR_REQUIRE(work == nullptr || (work_bytes >= gather_bytes(n_sites, m) &&
                                    reinterpret_cast<uintptr_t>(work) % 256 == 0),
                "density_backward: work must hold vgr_density_backward_work_size(N, m) = %lld bytes, 256-byte aligned",
                static_cast<long long>(gather_bytes(n_sites, m)));
    VGR_REQUIRE(work == nullptr || (m <= INT_MAX && n_sites <= int64_t(kScanTile) * kScanTile),
                "density_backward: with a workspace, m must be < 2^31 and N at most %lld",
                static_cast<long long>(int64_t(kScanTile) * kScanTile));
    const GradGraph g{points, offsets, adj, int(n_sites)};
    const GaussIn G{log_scale, reinterpret_cast<const float4*>(quat)};
    const hipStream_t st = as_stream(stream);
    if (work == nullptr) {
        hipLaunchKernelGGL(density_backward_kernel, dim3(grid_for(m, kBlock)), dim3(kBlock), 0, st, g, raw, G, x, site,
                           m, grad_sigma, g_raw, g_ls, g_quat);
        return launch_status("density_backward_kernel");
    }
    const GatherWork W = gather_work(work, n_sites, m);
    sort_samples<1>(g, site, grad_sigma, m, W.count, W.start, W.tile_sum, W.slot, st);
    float4* recs = static_cast<float4*>(W.recs);
    hipLaunchKernelGGL(density_record_kernel, dim3(grid_for(m, kBlock)), dim3(kBlock), 0, st, x, grad_sigma, m, W.slot,
                       recs);
    hipLaunchKernelGGL(density_gather_kernel, dim3(grid_for(n_sites, kBlock)), dim3(kBlock), 0, st, g, raw, G, W.start,
                       recs, g_raw, g_ls, g_quat);
    return launch_status("density_gather_kernel");
}

extern "C" int64_t vgr_color_backward_work_size(int64_t n_sites, int64_t m) {
    return n_sites > 0 && m >= 0 ? vgr::gather_bytes(n_sites, m) : 0;
}

extern "C" int vgr_color_backward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                                  int64_t n_adj, const float* log_scale, const float* quat, const float* sh,
                                  int64_t sh_deg, const float* x, const float* dirs, const int32_t* site, int64_t m,
                                  const float* rgb, const float* grad_rgb, float* g_ls, float* g_quat, float* g_sh,
                                  void* work, int64_t work_bytes, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(m >= 0, "color_backward: m must be >= 0");
    VGR_REQUIRE(sh_deg >= 0 && sh_deg <= 3, "sh_deg must be in [0, 3] (got %lld)", static_cast<long long>(sh_deg));
    if (m == 0) return VGR_OK;
    if (int rc = check_grad_graph("color_backward", points, n_sites, offsets, adj, n_adj)) return rc;
    VGR_REQUIRE(log_scale && quat && sh && x && dirs && site && rgb && grad_rgb && g_ls && g_quat && g_sh,
                "color_backward: null pointer");
    VGR_REQUIRE(work == nullptr || (work_bytes >= gather_bytes(n_sites, m) &&
                                    reinterpret_cast<uintptr_t>(work) % 256 == 0),
                "color_backward: work must hold vgr_color_backward_work_size(N, m) = %lld bytes, 256-byte aligned",
                static_cast<long long>(gather_bytes(n_sites, m)));
    VGR_REQUIRE(work == nullptr || (m <= INT_MAX && n_sites <= int64_t(kScanTile) * kScanTile),
                "color_backward: with a workspace, m must be < 2^31 and N at most %lld",
                static_cast<long long>(int64_t(kScanTile) * kScanTile));
    const GradGraph g{points, offsets, adj, int(n_sites)};
    const GaussIn H{log_scale, reinterpret_cast<const float4*>(quat)};
    const float4* s4 = reinterpret_cast<const float4*>(sh);
    const hipStream_t st = as_stream(stream);
    switch (sh_deg) {
        case 0: return color_backward_launch<0>(g, H, s4, x, dirs, site, m, rgb, grad_rgb, g_ls, g_quat, g_sh, work, st);
        case 1: return color_backward_launch<1>(g, H, s4, x, dirs, site, m, rgb, grad_rgb, g_ls, g_quat, g_sh, work, st);
        case 2: return color_backward_launch<2>(g, H, s4, x, dirs, site, m, rgb, grad_rgb, g_ls, g_quat, g_sh, work, st);
        default:
            return color_backward_launch<3>(g, H, s4, x, dirs, site, m, rgb, grad_rgb, g_ls, g_quat, g_sh, work, st);
    }
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
