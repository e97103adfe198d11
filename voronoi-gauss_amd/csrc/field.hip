// Forward field operators of the NeRF-style path, gfx950: greedy walk of sorted samples, density and colour
// at samples over the Voronoi neighbourhood, and conics from (log_scale, quat).
//
// Semantics follow csrc/vgf.cu of the reference: walk_kernel :51-79 (strict <, so the first closer neighbour
// in CSR order wins), gauss_local :98-119 and density_forward_kernel :163-177, sh_eval/unit_dir/
// color_forward_kernel :230-282 (online softmax), conic_local/conic_forward_kernel :350-380.
//
// MI355X layouts:
// - walk: a group of 16 lanes (one DPP row) per ray. The group holds the neighbourhood of the ray's current site in
//   registers (lane g: entries g, g + 16, g + 32, g + 48) and streams the ray's samples through it: a sample that
//   stays in the site costs a distance per held entry and a four-step row butterfly, no memory access; only a move
//   reloads. The first-found rule of the sequential scan is the lexicographic minimum of (distance, CSR position),
//   which the butterfly computes in any order, so sites and step counts are those of a sequential scan.
// - density: one sample per lane over per-site Gaussian records built once per call (gauss_pack_kernel).
// - colour: below 2^22 samples a group of 4 lanes per sample (16 samples per wave): lane g blends the entries
//   g, g + 4, ... of the neighbourhood into a partial online softmax (its own running minimum), and the group merges
//   the partials in a butterfly, so that a small batch still fills the GPU; from 2^22 samples one lane per sample
//   blends its whole neighbourhood (no merges).
// - conic: one site per lane.
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

// ------------------------------------------------------------------ walk: 16 lanes per ray
constexpr int kWalkLanes = 16;  // one DPP row per ray, 4 rays per wave
constexpr int kWalkHeld = 4;    // neighbourhood entries each lane keeps in registers (64 per group)

// Squared distance from x to p, summed in the reference's order (no contraction: bit-exact walks).
__device__ __forceinline__ float sq_dist(float px, float py, float pz, const float (&x)[3]) {
    const float a = x[0] - px, b = x[1] - py, c = x[2] - pz;
    return a * a + b * b + c * c;
}

// Candidate (d, e, k): keeps the lexicographic minimum of (distance, CSR position), i.e. the entry a sequential scan
// with a strict < would keep.
__device__ __forceinline__ void keep_first_closest(float d, int e, int k, float& bd, int& be, int& bk) {
    if (d < bd || (d == bd && e < be)) bd = d, be = e, bk = k;
}

template <int CTRL>
__device__ __forceinline__ void first_closest_step(float& bd, int& be, int& bk) {
    keep_first_closest(row_perm<CTRL>(bd), row_perm<CTRL>(be), row_perm<CTRL>(bk), bd, be, bk);
}

// The neighbourhood of one site as a group of 16 lanes holds it: lane g keeps entries g + 16 j (j < kWalkHeld) as
// (position, site); entries beyond 64 stay in memory and are read by the same lanes in every scan.
struct HeldCell {
    int site, e0, e1;
    float px[kWalkHeld], py[kWalkHeld], pz[kWalkHeld];
    int k[kWalkHeld];
};

__device__ __forceinline__ void hold_cell(const Graph& g, int c, int lane, HeldCell& H) {
    H.site = c;
    H.e0 = g.offsets[c], H.e1 = g.offsets[c + 1];
#pragma unroll
    for (int j = 0; j < kWalkHeld; ++j) {
        const int e = H.e0 + lane + kWalkLanes * j;
        H.k[j] = e < H.e1 ? g.adj[e] : -1;
    }
#pragma unroll
    for (int j = 0; j < kWalkHeld; ++j) {
        const int64_t q = 3 * static_cast<int64_t>(H.k[j] >= 0 ? H.k[j] : c);
        H.px[j] = g.points[q], H.py[j] = g.points[q + 1], H.pz[j] = g.points[q + 2];
    }
}

// One scan of the held site's neighbourhood for the point x: the site a sequential strict-< scan started from
// best_d would move to (best_d updated), or the held site itself.
__device__ __forceinline__ int scan_held(const Graph& g, const HeldCell& H, int lane, const float (&x)[3],
                                         float& best_d) {
    float bd = best_d;
    int be = -1, bk = H.site;  // staying wins ties: a neighbour must be strictly closer
#pragma unroll
    for (int j = 0; j < kWalkHeld; ++j)
        if (H.k[j] >= 0) keep_first_closest(sq_dist(H.px[j], H.py[j], H.pz[j], x), H.e0 + lane + kWalkLanes * j,
                                            H.k[j], bd, be, bk);
    for (int e = H.e0 + lane + kWalkLanes * kWalkHeld; e < H.e1; e += kWalkLanes) {  // cells beyond 64 entries
        const int q = g.adj[e];
        const int64_t q3 = 3 * static_cast<int64_t>(q);
        keep_first_closest(sq_dist(g.points[q3], g.points[q3 + 1], g.points[q3 + 2], x), e, q, bd, be, bk);
    }
    first_closest_step<kXor1>(bd, be, bk);
    first_closest_step<kXor2>(bd, be, bk);
    first_closest_step<kHalfMirror>(bd, be, bk);
    first_closest_step<kMirror>(bd, be, bk);
    best_d = bd;
    return bk;
}

// Every sample of ray r (S sorted parameters in z) walked from the previous sample's site; the group's lanes hold
// the same values throughout, lane g stores the sites of samples g, g + 16, ... (16 consecutive ints per store).
__global__ void __launch_bounds__(kBlock)
    walk_group_kernel(Graph g, const float* __restrict__ o, const float* __restrict__ d, const float* __restrict__ z,
                      const int* __restrict__ start, int64_t B, int S, int* __restrict__ site,
                      int* __restrict__ steps) {
    const int lane = static_cast<int>(threadIdx.x) % kWalkLanes;
    const int64_t r = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) / kWalkLanes;
    if (r >= B) return;  // whole groups leave together
    int* out = site + r * S;
    const int first = start[r];
    if (first < 0 || first >= g.n_sites) {  // invalid start: every sample unresolved
        for (int s = lane; s < S; s += kWalkLanes) out[s] = -1;
        if (steps != nullptr && lane == 0) steps[r] = 0;
        return;
    }
    const float org[3] = {o[3 * r], o[3 * r + 1], o[3 * r + 2]}, dir[3] = {d[3 * r], d[3 * r + 1], d[3 * r + 2]};
    HeldCell H;
    hold_cell(g, first, lane, H);
    int64_t cur3 = 3 * static_cast<int64_t>(first);
    float cx = g.points[cur3], cy = g.points[cur3 + 1], cz = g.points[cur3 + 2];
    int moves = 0, mine = -1;
    for (int s = 0; s < S; ++s) {
        const float t = z[r * S + s];
        const float x[3] = {org[0] + t * dir[0], org[1] + t * dir[1], org[2] + t * dir[2]};
        float best_d = sq_dist(cx, cy, cz, x);
        for (int it = 0; it < kWalkCap; ++it) {
            const int next = scan_held(g, H, lane, x, best_d);
            if (next == H.site) break;
            ++moves;
            hold_cell(g, next, lane, H);
            cur3 = 3 * static_cast<int64_t>(next);
            cx = g.points[cur3], cy = g.points[cur3 + 1], cz = g.points[cur3 + 2];
        }
        const int slot = s % kWalkLanes;
        if (slot == lane) mine = H.site;
        if (slot == kWalkLanes - 1 || s == S - 1) {
            if (lane <= slot) out[s - slot + lane] = mine;
        }
    }
    if (steps != nullptr && lane == 0) steps[r] = moves;
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

// ------------------------------------------------------------------ colour: 1 or 4 lanes per sample
// Lanes per sample by batch size: below kColourWide samples a lane per sample would leave the GPU's 256 CUs short of
// waves, so 4 lanes share a sample's neighbourhood; above it one lane per sample skips the group merges.
constexpr int64_t kColourWide = int64_t(1) << 22;
__host__ __device__ constexpr int colour_lanes(int64_t m) { return m >= kColourWide ? 1 : 4; }

// Partial online softmax of a lane's share of the neighbourhood: running minimum m of the Mahalanobis distances, and
// sum a of exp(-(m_k - m) / 2) and of those weights times the clamped colours.
struct Softmax {
    float m, a, r, g, b;
};

__device__ __forceinline__ void softmax_add(Softmax& P, float mk, const float (&c)[3]) {
    if (mk < P.m) {  // rescale to the new minimum (the first term: everything is 0 and exp(-inf) = 0)
        const float f = fexp(-0.5f * (P.m - mk));
        P.a *= f, P.r *= f, P.g *= f, P.b *= f;
        P.m = mk;
    }
    const float w = fexp(-0.5f * (mk - P.m));
    P.a += w;
    P.r += w * fmaxf(c[0], 0.f), P.g += w * fmaxf(c[1], 0.f), P.b += w * fmaxf(c[2], 0.f);
}

// Merges the partial of the lane CTRL pairs this one with: both rescaled to the smaller minimum, products rounded
// separately so that both lanes of a pair compute the same bits.
template <int CTRL>
__device__ __forceinline__ void softmax_merge(Softmax& P) {
    const Softmax Q{row_perm<CTRL>(P.m), row_perm<CTRL>(P.a), row_perm<CTRL>(P.r), row_perm<CTRL>(P.g),
                    row_perm<CTRL>(P.b)};
    const float m = fminf(P.m, Q.m);
    const float fp = fexp(-0.5f * (P.m - m)), fq = fexp(-0.5f * (Q.m - m));
    const float a1 = P.a * fp, a2 = Q.a * fq, r1 = P.r * fp, r2 = Q.r * fq;
    const float g1 = P.g * fp, g2 = Q.g * fq, b1 = P.b * fp, b2 = Q.b * fq;
    P.m = m, P.a = a1 + a2, P.r = r1 + r2, P.g = g1 + g2, P.b = b1 + b2;
}

// SH_k(d) + 1/2 over the coefficients of degree <= DEG (coefficient j of channel c at 3 j + c of the row).
template <int DEG>
__device__ __forceinline__ void sh_colour(const float4* __restrict__ row, const float (&b)[16], float (&c)[3]) {
    constexpr int nb = (DEG + 1) * (DEG + 1), nv = sh_vec4_f32(DEG);
    float4 f[nv];
#pragma unroll
    for (int q = 0; q < nv; ++q) f[q] = row[q];  // the whole row in flight before the first product
    c[0] = c[1] = c[2] = 0.5f;
#pragma unroll
    for (int q = 0; q < nv; ++q) {
        const float fv[4] = {f[q].x, f[q].y, f[q].z, f[q].w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = 4 * q + u;
            if (j / 3 < nb) c[j % 3] += b[j / 3] * fv[u];
        }
    }
}

// Colour at sample t: the normalised blend of max(SH_k(d) + 1/2, 0) over k in {i} U adj(i) with weights
// exp(-(m_k - m_min) / 2). REC: m_k from the per-site records (gauss_pack_kernel), else from (log_scale, quat).
// L lanes per sample (1 or 4): lane l takes positions l, l + L, ... of the neighbourhood.
template <int DEG, bool REC, int L>
__global__ void __launch_bounds__(kBlock)
    colour_group_kernel(Graph g, Gauss H, const float4* __restrict__ rec, const float4* __restrict__ sh,
                        const float* __restrict__ x, const float* __restrict__ dirs, const int* __restrict__ site,
                        int64_t m, float* __restrict__ rgb) {
    static_assert(L == 1 || L == 4, "lanes per sample");
    const int lane = static_cast<int>(threadIdx.x) % L;
    const int64_t t = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) / L;
    if (t >= m) return;  // whole groups leave together
    const int i = site[t];
    if (i < 0 || i >= g.n_sites) {
        for (int c = lane; c < 3; c += L) rgb[3 * t + c] = 0.f;
        return;
    }
    const float px = x[3 * t], py = x[3 * t + 1], pz = x[3 * t + 2];
    float u[3] = {dirs[3 * t], dirs[3 * t + 1], dirs[3 * t + 2]};
    const float inv = rsqrtf(fmaxf(u[0] * u[0] + u[1] * u[1] + u[2] * u[2], 1e-20f));
    u[0] *= inv, u[1] *= inv, u[2] *= inv;
    float b[16];
    sh_basis(u[0], u[1], u[2], DEG, b);
    Softmax P{kInf, 0.f, 0.f, 0.f, 0.f};
    const int e0 = g.offsets[i], e1 = g.offsets[i + 1];
    for (int e = e0 - 1 + lane; e < e1; e += L) {  // position e0 - 1 stands for the site itself
        const int k = e < e0 ? i : g.adj[e];
        float mk;
        if constexpr (REC) {
            float raw_c;
            mk = gauss_m_rec(rec, k, px, py, pz, raw_c);
        } else {
            mk = gauss_m(g, H, k, px, py, pz, 1.f);
        }
        float c[3];
        sh_colour<DEG>(sh + 12 * static_cast<int64_t>(k), b, c);
        softmax_add(P, mk, c);
    }
    if constexpr (L == 4) {
        softmax_merge<kXor1>(P);
        softmax_merge<kXor2>(P);
    }
    for (int c = lane; c < 3; c += L) rgb[3 * t + c] = (c == 0 ? P.r : (c == 1 ? P.g : P.b)) / P.a;
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

template <int DEG, int L>
void launch_colour_l(bool rec, hipStream_t st, const Graph& g, const Gauss& H, const float4* R, const float4* sh,
                     const float* x, const float* dirs, const int* site, int64_t m, float* rgb) {
    const dim3 grid(grid_for(m * L, kBlock));
    if (rec)
        hipLaunchKernelGGL((colour_group_kernel<DEG, true, L>), grid, dim3(kBlock), 0, st, g, H, R, sh, x, dirs, site,
                           m, rgb);
    else
        hipLaunchKernelGGL((colour_group_kernel<DEG, false, L>), grid, dim3(kBlock), 0, st, g, H, R, sh, x, dirs, site,
                           m, rgb);
}

template <int DEG>
void launch_colour(bool rec, hipStream_t st, const Graph& g, const Gauss& H, const float4* R, const float4* sh,
                   const float* x, const float* dirs, const int* site, int64_t m, float* rgb) {
    if (colour_lanes(m) == 1)
        launch_colour_l<DEG, 1>(rec, st, g, H, R, sh, x, dirs, site, m, rgb);
    else
        launch_colour_l<DEG, 4>(rec, st, g, H, R, sh, x, dirs, site, m, rgb);
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
    VGR_REQUIRE(n_rays <= INT64_MAX / kWalkLanes, "walk: n_rays too large");
    hipLaunchKernelGGL(walk_group_kernel, dim3(grid_for(n_rays * kWalkLanes, kBlock)), dim3(kBlock), 0,
                       as_stream(stream), Graph{points, offsets, adj, int(n_sites)}, o, d, z, start, n_rays,
                       int(n_samples), site, steps);
    return launch_status("walk_group_kernel");
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
    const dim3 block(kBlock);
    const hipStream_t st = as_stream(stream);
    const bool rec = use_records(work, work_bytes, n_sites, m);
    const float4* R = static_cast<const float4*>(work);
    if (rec)
        hipLaunchKernelGGL(gauss_pack_kernel, dim3(grid_for(n_sites, kBlock)), block, 0, st, g, H, nullptr, 1.f,
                           static_cast<float4*>(work));
    switch (sh_deg) {
        case 0: launch_colour<0>(rec, st, g, H, R, s4, x, dirs, site, m, rgb); break;
        case 1: launch_colour<1>(rec, st, g, H, R, s4, x, dirs, site, m, rgb); break;
        case 2: launch_colour<2>(rec, st, g, H, R, s4, x, dirs, site, m, rgb); break;
        default: launch_colour<3>(rec, st, g, H, R, s4, x, dirs, site, m, rgb); break;
    }
    return launch_status("colour_group_kernel");
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
