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
// shuffle reductions become sequential per-lane sums. Per sample, one fused pass over the neighbourhood does the
// walk's test, the density and the colour minimum for several consecutive samples at once; the colour blends of the
// coloured samples of a cell share one pass, which evaluates each neighbour's SH colour once for all of them.
//
// Site blocks: a pack kernel first gathers each site's point, min(raw, 30), density conic, colour conic and SH
// coefficients into one line-aligned block: the 64-byte record and the first 64 bytes of SH fill one 128-byte line,
// the rest of the SH the next. Incoherent rays fetch a fresh line per lane for every neighbour: a neighbourhood pass
// then costs one line per neighbour (the record), a colour pass two (one when sh_deg <= 1), instead of one line per
// scattered array.
#include "vgr_abi.h"
#include "vgr_device.h"

namespace vgr {
namespace {

constexpr int kBlock = 64;

// Site block k = rec[BLK k .. BLK k + BLK - 1] (float4): the record (p_k, min(raw_k, 30)), (dA_k[0..3]),
// (dA_k[4..5], cA_k[0..1]), (cA_k[2..5]), then the first NV float4 of the site's SH row (N, 16, 3); BLK = 8 (one
// 128-byte line) when they fit, else 16.
constexpr int kRec = 4;
__host__ __device__ constexpr int block_vec4(int nv) { return kRec + nv <= 8 ? 8 : 16; }

struct MarchField {
    const float4* __restrict__ rec;  // (N, BLK)
    const int* __restrict__ offsets;  // (N + 1)
    const int* __restrict__ adj;      // (M)
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
    const int* __restrict__ order;  // processing order of the rays (a permutation of 0 .. n - 1), or null
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

// One lane per float4 of the blocks (the record's four, then the SH row's nv), so that a wave's stores are
// consecutive 16-byte pieces of consecutive blocks.
__global__ void __launch_bounds__(256)
    march_pack_kernel(const float* __restrict__ points, const float* __restrict__ raw, const float* __restrict__ dA,
                      const float* __restrict__ cA, const float4* __restrict__ sh, int nv, int blk, int64_t n,
                      float4* __restrict__ rec) {
    const int per = kRec + nv;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n * per) return;
    const int64_t k = i / per;
    const int q = static_cast<int>(i - k * per);
    const float* a = dA + 6 * k;
    const float* c = cA + 6 * k;
    float4 v;
    if (q == 0) {
        const float* p = points + 3 * k;
        v = make_float4(p[0], p[1], p[2], fminf(raw[k], 30.f));
    } else if (q == 1) {
        v = make_float4(a[0], a[1], a[2], a[3]);
    } else if (q == 2) {
        v = make_float4(a[4], a[5], c[0], c[1]);
    } else if (q == 3) {
        v = make_float4(c[2], c[3], c[4], c[5]);
    } else {
        v = sh[12 * k + (q - kRec)];
    }
    rec[blk * k + q] = v;
}

void launch_pack(const float* points, const float* raw, const float* dA, const float* cA, const float* sh, int64_t n,
                 int64_t sh_deg, float4* rec, hipStream_t s) {
    const int nv = sh_vec4_f32(static_cast<int>(sh_deg));
    hipLaunchKernelGGL(march_pack_kernel, dim3(grid_for(n * (kRec + nv), 256)), dim3(256), 0, s, points, raw, dA, cA,
                       reinterpret_cast<const float4*>(sh), nv, block_vec4(nv), n, rec);
}

struct SiteRec {
    float4 q0, q1, q2, q3;
};

template <int BLK>
__device__ __forceinline__ SiteRec site_rec(const MarchField& F, int k) {
    const float4* r = F.rec + BLK * static_cast<int64_t>(k);
    return {r[0], r[1], r[2], r[3]};
}

__device__ __forceinline__ void offset_to(const float4& p, const float (&x)[3], float (&v)[3]) {
    v[0] = x[0] - p.x, v[1] = x[1] - p.y, v[2] = x[2] - p.z;
}

// Mahalanobis terms v^T A v of the density and colour conics of a record.
__device__ __forceinline__ float density_m(const SiteRec& R, const float (&v)[3]) {
    return maha(R.q1.x, R.q1.y, R.q1.z, R.q1.w, R.q2.x, R.q2.y, v[0], v[1], v[2]);
}
__device__ __forceinline__ float color_m(const float4& c0, const float4& c1, const float (&v)[3]) {
    return maha(c0.z, c0.w, c1.x, c1.y, c1.z, c1.w, v[0], v[1], v[2]);
}

// 1/2 + sum_{j < (deg+1)^2} b_j sh_kj per channel, reading only the float4 that hold those coefficients, CHUNK
// float4 at a time (the scheduling barrier keeps the next chunk's loads from being hoisted, which bounds the
// registers the loads occupy; CHUNK = NV requests the whole row at once).
constexpr int kShChunk = 4;

template <int NV, int CHUNK = kShChunk>
__device__ __forceinline__ void sh_eval_n(const float4* __restrict__ s, const float (&b)[16], int nb, float (&c)[3]) {
    c[0] = c[1] = c[2] = 0.5f;
#pragma unroll
    for (int q0 = 0; q0 < NV; q0 += CHUNK) {
        float4 f[CHUNK];
#pragma unroll
        for (int q = 0; q < CHUNK; ++q)
            if (q0 + q < NV) f[q] = s[q0 + q];
#pragma unroll
        for (int q = 0; q < CHUNK; ++q) {
            if (q0 + q < NV) {
                const float fv[4] = {f[q].x, f[q].y, f[q].z, f[q].w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int i = 4 * (q0 + q) + u;
                    if (i / 3 < nb) c[i % 3] += b[i / 3] * fv[u];
                }
            }
        }
        if (q0 + CHUNK < NV) __builtin_amdgcn_sched_barrier(0);
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

// Samples are resolved several at a time: one pass over the neighbourhood {i} U adj(i) of site i evaluates, for
// each of the next sample points x_j, the lexicographic argmin of (|x_j - p_k|^2, k) (the greedy walk's test), the
// density sum and the colour terms. Sample j + 1's walk starts at sample j's site, so every leading sample at which i
// wins is resolved by this one pass exactly as by a pass of its own (same neighbours, same order, same roundings);
// the first sample at which i loses walks on from its argmin, and the pass at the next site covers it and the
// samples after it. Each quantity accumulates over the neighbours in the same order as the reference's separate
// passes. The backward's pass (cell_pass, kBatch samples) takes the smallest colour Mahalanobis distance of each
// sample, for a colour pass of its own; the forward's (fwd_pass below) blends the colours in the same pass.
constexpr int kBatch = 6;

struct CellPass {
    int best[kBatch];
    float sigma[kBatch], mmin[kBatch];
};

// x = o + t d, rounded per operation (the product, then the sum).
__device__ __forceinline__ void point_at(const float (&o)[3], const float (&d)[3], float t, float (&x)[3]) {
#pragma unroll
    for (int a = 0; a < 3; ++a) x[a] = o[a] + t * d[a];
}

template <int BLK>
__device__ void cell_pass(const MarchField& F, int i, const float (&o)[3], const float (&d)[3],
                          const float (&t)[kBatch], CellPass& R) {
    const int e0 = F.offsets[i], n = F.offsets[i + 1] - e0 + 1;
    float bd[kBatch], s[kBatch], mm[kBatch];
    int bk[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) bd[j] = kInf, s[j] = 0.f, mm[j] = kInf, bk[j] = INT_MAX;
    int k = i;
    int kn = neighbor(F, i, e0, min(1, n - 1));
    for (int e = 0; e < n; ++e) {
        const int k2 = neighbor(F, i, e0, min(e + 2, n - 1));  // in flight: the neighbour after next
        const SiteRec rc = site_rec<BLK>(F, k);
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            float x[3], v[3];
            float tj = t[j];
            asm volatile("" : "+v"(tj));  // recompute x per neighbour: 3 fewer live registers per sample
            point_at(o, d, tj, x);
            offset_to(rc.q0, x, v);
            const float dk = v[0] * v[0] + v[1] * v[1] + v[2] * v[2];
            if (dk < bd[j] || (dk == bd[j] && k < bk[j])) bd[j] = dk, bk[j] = k;
            s[j] += fexp(rc.q0.w - 0.5f * density_m(rc, v));
            mm[j] = fminf(mm[j], color_m(rc.q2, rc.q3, v));
        }
        k = kn, kn = k2;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) R.best[j] = bk[j], R.sigma[j] = s[j], R.mmin[j] = mm[j];
}

// The forward's pass: kFwd samples, their walk tests and densities as in cell_pass, and each sample's colour blend
// in the same pass, so that a neighbour's block (its record line and SH line) is read once per cell visit, where a
// separate colour pass would fetch the record line again (3 random lines per neighbour of a coloured visit, now 2).
// Each sample keeps a running blend relative to its smallest colour Mahalanobis distance so far, m: the sums of
// exp(-(m_k - m) / 2) and of those weights times the colours max(SH_k(d) + 1/2, 0), both rescaled by
// exp(-(m_old - m_new) / 2) when m falls, which after the pass is the normalised blend with weights
// exp(-(m_k - m_min) / 2) up to rounding. Samples past the first that walks on are blended for nothing; the next pass
// redoes them.
//
// Registers: the blend sums of the samples (a float4 each) and the ray's SH basis live in the wave's LDS, one float4
// per lane per row (consecutive lanes, consecutive 16 bytes: no bank conflicts); a neighbour's 12 SH float4 are
// requested with its record, one round trip per neighbour. kFwd = 8 at 3 waves per SIMD.
constexpr int kFwd = 8;
constexpr int kFwdWaves = 3;
constexpr int kFwdLds = 4 + kFwd;  // float4 rows per lane: the basis (4), then the samples' sums

struct FwdPass {
    int best[kFwd];
    float sigma[kFwd];
    float4 blend[kFwd];  // (sum a, sum a r, sum a g, sum a b)
};

// lds: this lane's first row; row q at lds[kBlock q].
template <int BLK, int NV>
__device__ void fwd_pass(const MarchField& F, int i, const float (&o)[3], const float (&d)[3],
                         const float (&t)[kFwd], float4* lds, FwdPass& R) {
    const int e0 = F.offsets[i], n = F.offsets[i + 1] - e0 + 1;
    const int nb = (F.sh_deg + 1) * (F.sh_deg + 1);
    float4* sums = lds + 4 * kBlock;
    float bd[kFwd], s[kFwd], mm[kFwd];
    int bk[kFwd];
#pragma unroll
    for (int j = 0; j < kFwd; ++j) {
        bd[j] = kInf, s[j] = 0.f, mm[j] = kInf, bk[j] = INT_MAX;
        sums[kBlock * j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    int k = i;
    int kn = neighbor(F, i, e0, min(1, n - 1));
    for (int e = 0; e < n; ++e) {
        const int k2 = neighbor(F, i, e0, min(e + 2, n - 1));  // in flight: the neighbour after next
        const float4* blk = F.rec + BLK * static_cast<int64_t>(k);
        const SiteRec rc = {blk[0], blk[1], blk[2], blk[3]};
        float c[3];
        {
            float b[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = lds[kBlock * q];
                b[4 * q] = v.x, b[4 * q + 1] = v.y, b[4 * q + 2] = v.z, b[4 * q + 3] = v.w;
            }
            sh_eval_n<NV, NV>(blk + kRec, b, nb, c);
        }
        c[0] = fmaxf(c[0], 0.f), c[1] = fmaxf(c[1], 0.f), c[2] = fmaxf(c[2], 0.f);
#pragma unroll
        for (int j = 0; j < kFwd; ++j) {
            float x[3], v[3];
            float tj = t[j];
            asm volatile("" : "+v"(tj));  // recompute x per neighbour: 3 fewer live registers per sample
            point_at(o, d, tj, x);
            offset_to(rc.q0, x, v);
            const float dk = v[0] * v[0] + v[1] * v[1] + v[2] * v[2];
            if (dk < bd[j] || (dk == bd[j] && k < bk[j])) bd[j] = dk, bk[j] = k;
            s[j] += fexp(rc.q0.w - 0.5f * density_m(rc, v));
            const float mc = color_m(rc.q2, rc.q3, v);
            const bool lower = mc < mm[j];  // a new minimum: the sums so far scale down, this term weighs 1
            const float ex = fexp(-0.5f * (lower ? mm[j] - mc : mc - mm[j]));
            const float keep = lower ? ex : 1.f, add = lower ? 1.f : ex;
            float4 a = sums[kBlock * j];
            a.x = a.x * keep + add;
            a.y = a.y * keep + add * c[0], a.z = a.z * keep + add * c[1], a.w = a.w * keep + add * c[2];
            sums[kBlock * j] = a;
            mm[j] = fminf(mm[j], mc);
        }
        k = kn, kn = k2;
    }
#pragma unroll
    for (int j = 0; j < kFwd; ++j) R.best[j] = bk[j], R.sigma[j] = s[j], R.blend[j] = sums[kBlock * j];
}

template <int NV, bool TRACE>
__device__ void march_ray(const MarchField& F, const MarchParams& M, const MarchRays& R, const MarchOut& O, int64_t r,
                          int cur, float4* lds) {
    const float o[3] = {R.o[3 * r], R.o[3 * r + 1], R.o[3 * r + 2]};
    const float d[3] = {R.d[3 * r], R.d[3 * r + 1], R.d[3 * r + 2]};
    const float near = R.t_near[r], mid = R.t_mid[r], far = R.t_far[r];
    const int n_in = mid > near ? static_cast<int>(ceilf((mid - near) / M.dt)) : 0;
    const int n_total = n_in + M.n_bg;
    {  // the ray's SH basis, read by every colour evaluation of its passes
        float b[16];
        sh_basis(d[0], d[1], d[2], F.sh_deg, b);
#pragma unroll
        for (int q = 0; q < 4; ++q) lds[kBlock * q] = make_float4(b[4 * q], b[4 * q + 1], b[4 * q + 2], b[4 * q + 3]);
    }
    int n_samples = 0, n_color = 0, walk_steps = 0;
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f}, dep = 0.f;
    // k: first unresolved sample; moves: greedy-walk steps taken so far for sample k
    int k = 0, moves = 0;
    bool live = true;
    while (live && k < n_total) {
        float ts[kFwd];
#pragma unroll
        for (int j = 0; j < kFwd; ++j) {
            float unused;
            sample_at(near, mid, far, n_in, M, min(k + j, n_total - 1), ts[j], unused);
        }
        FwdPass C;
        fwd_pass<block_vec4(NV), NV>(F, cur, o, d, ts, lds, C);
        // walk bound reached: the sample takes the current site, unverified
        const bool force = moves >= kWalkCap;
        int nres = 0, next = cur;
        bool run = true;
#pragma unroll
        for (int j = 0; j < kFwd; ++j) {
            if (!run || k + j >= n_total) {
                run = false;
            } else if (C.best[j] == cur || (j == 0 && force)) {
                if (TRACE && n_samples < O.trace_cap) O.trace[r * O.trace_cap + n_samples] = cur;
                float t, delta;
                sample_at(near, mid, far, n_in, M, k + j, t, delta);
                const float alpha = 1.f - fexp(-C.sigma[j] * delta);
                const float w = T * alpha;
                ++n_samples, ++nres;
                if (w > M.w_thresh) {
                    const float inv_a = 1.f / C.blend[j].x;
                    const float Cs[3] = {C.blend[j].y * inv_a, C.blend[j].z * inv_a, C.blend[j].w * inv_a};
#pragma unroll
                    for (int a = 0; a < 3; ++a) acc[a] += w * Cs[a];
                    dep += w * t;
                    ++n_color;
                }
                T *= 1.f - alpha;
                if (T < M.t_thresh) run = live = false;
            } else {
                next = C.best[j], run = false;
            }
        }
        k += nres;
        moves = nres > 0 ? 0 : moves;
        if (live && k < n_total && next != cur) cur = next, ++walk_steps, ++moves;
    }
#pragma unroll
    for (int a = 0; a < 3; ++a) O.rgb[3 * r + a] = acc[a];
    O.T[r] = T;
    O.depth[r] = dep;
    O.stats[3 * r] = n_samples, O.stats[3 * r + 1] = n_color, O.stats[3 * r + 2] = walk_steps;
}

template <bool TRACE>
__global__ void __launch_bounds__(kBlock, kFwdWaves)
    march_forward_kernel(MarchField F, MarchParams M, MarchRays R, MarchOut O) {
    __shared__ float4 fwd_lds[kFwdLds * kBlock];
    const int64_t i = xcd_block_id() * kBlock + threadIdx.x;
    if (i >= R.n) return;
    const int64_t r = R.order != nullptr ? R.order[i] : i;
    if (r < 0 || r >= R.n) return;  // not a permutation entry: nothing is read or written
    const int cur = R.start[r];
    if (cur < 0 || cur >= F.n_sites) {  // not traced: empty foreground
        O.rgb[3 * r] = O.rgb[3 * r + 1] = O.rgb[3 * r + 2] = 0.f;
        O.T[r] = 1.f, O.depth[r] = 0.f;
        O.stats[3 * r] = O.stats[3 * r + 1] = O.stats[3 * r + 2] = 0;
        return;
    }
    switch (F.sh_deg) {
        case 0: march_ray<sh_vec4_f32(0), TRACE>(F, M, R, O, r, cur, fwd_lds + threadIdx.x); break;
        case 1: march_ray<sh_vec4_f32(1), TRACE>(F, M, R, O, r, cur, fwd_lds + threadIdx.x); break;
        case 2: march_ray<sh_vec4_f32(2), TRACE>(F, M, R, O, r, cur, fwd_lds + threadIdx.x); break;
        default: march_ray<sh_vec4_f32(3), TRACE>(F, M, R, O, r, cur, fwd_lds + threadIdx.x); break;
    }
}

// ------------------------------------------------------------------------------------------------- backward
//
// The backward re-marches every ray (march.cu:264-345): the same batched neighbourhood passes resolve the same
// samples at the same sites, a colour pass blends the coloured samples of each pass as the forward does, and then
// the upstream gradient of each resolved sample's density, d rgb / d sigma = delta (T_next C - (rgb - acc)) and
// d T / d sigma = -delta T (acc: the colour composited up to and including the sample), and of its colour, w dL/drgb,
// are pushed to the neighbourhood. All samples of a pass share one neighbourhood, so one more pass over it sums every
// sample's contribution per neighbour in registers and issues one set of fp32 atomics per neighbour and pass (1 for
// raw, 6 + 6 for the conics, 3 (deg + 1)^2 for the SH row) where the reference issues one per sample and neighbour.
// Per pair the reference's cut-offs hold: density terms with |g| <= 1e-12 and normalised colour weights below 1e-7
// contribute nothing. The SH gradient of a neighbour is b_j gR_c sum_s a_s w_s over the samples whose weight passes
// the cut-off, for the channels whose unclamped colour is positive (the colour depends only on the site and the ray).

struct MarchGradIn {
    const float* __restrict__ rgb;    // (B, 3) the forward's colour
    const float* __restrict__ T;      // (B) the forward's final transmittance
    const float* __restrict__ g_rgb;  // (B, 3)
    const float* __restrict__ g_T;    // (B)
};

// Gradients accumulate per site in one 256-byte block (two 128-byte lines) of the workspace: float 0 raw, 1..6 the
// density conic, 7..12 the colour conic, 16..63 the SH row (16, 3). One neighbour's atomics then touch one line (two
// above SH degree 1) instead of a line in each of four arrays; a final pass copies the blocks to the outputs.
constexpr int kGradBlock = 64;  // floats per site
constexpr int kGradSh = 16;

struct MarchGradOut {
    float* __restrict__ block;  // (N, 64)
};

// Copies the gradient blocks to g_raw (N), g_dA (N, 6), g_cA (N, 6) and g_sh (N, 16, 3): one lane per block float
// (contiguous reads; the stores of a block's density-conic, colour-conic and SH floats are contiguous too).
__global__ void __launch_bounds__(256)
    grad_unpack_kernel(const float* __restrict__ block, int64_t n, float* __restrict__ g_raw,
                       float* __restrict__ g_dA, float* __restrict__ g_cA, float* __restrict__ g_sh) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= kGradBlock * n) return;
    const int64_t k = i / kGradBlock;
    const int t = static_cast<int>(i - k * kGradBlock);
    const float v = block[i];
    if (t == 0)
        g_raw[k] = v;
    else if (t < 7)
        g_dA[6 * k + t - 1] = v;
    else if (t < 13)
        g_cA[6 * k + t - 7] = v;
    else if (t >= kGradSh)
        g_sh[48 * k + t - kGradSh] = v;
}

constexpr float kMinColourWeight = 1e-7f;
constexpr float kMinDensityGrad = 1e-12f;

// g += s (v v^T) in the packed symmetric layout of the conics (xx, 2xy, 2xz, yy, 2yz, zz).
__device__ __forceinline__ void add_outer(float (&g)[6], float s, const float (&v)[3]) {
    g[0] += s * v[0] * v[0];
    g[1] += 2.f * s * v[0] * v[1];
    g[2] += 2.f * s * v[0] * v[2];
    g[3] += s * v[1] * v[1];
    g[4] += 2.f * s * v[1] * v[2];
    g[5] += s * v[2] * v[2];
}

// The resolved samples of one pass: positions, density gradients, compositing weights, m_min, 1 / sum of shifted
// colour weights and gR . C; bit j of `coloured` marks a sample with w > w_thresh.
struct GradBatch {
    float t[kBatch], gsig[kBatch], w[kBatch], mmin[kBatch], inv_a[kBatch], grc[kBatch];
    int n;
    unsigned coloured;
};

// The gradient contributions of the resolved samples of a pass to neighbour k (record rc): raw, density conic,
// colour conic, and the SH factors gR_c sum_s a_s w_s for the channels whose unclamped colour is positive.
struct NeighbourGrad {
    float raw, dA[6], cA[6], sh[3];
    bool dens, col;
};

template <int NV>
__device__ __forceinline__ void neighbour_grad(const MarchField& F, int k, const float (&o)[3], const float (&d)[3],
                                               const float (&b)[16], int nb, const float (&gR)[3],
                                               const GradBatch& S, NeighbourGrad& N) {
    const float4* rp = F.rec + block_vec4(NV) * static_cast<int64_t>(k);
    const SiteRec rc = {rp[0], rp[1], rp[2], rp[3]};
    float c[3] = {0.f, 0.f, 0.f};
    if (S.coloured) sh_eval_n<NV>(rp + kRec, b, nb, c);
    const float gc3 = gR[0] * fmaxf(c[0], 0.f) + gR[1] * fmaxf(c[1], 0.f) + gR[2] * fmaxf(c[2], 0.f);
    float aw = 0.f;
    N.raw = 0.f;
#pragma unroll
    for (int u = 0; u < 6; ++u) N.dA[u] = N.cA[u] = 0.f;
    N.dens = N.col = false;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
        if (j < S.n) {
            float x[3], v[3];
            point_at(o, d, S.t[j], x);
            offset_to(rc.q0, x, v);
            if (S.gsig[j] != 0.f) {
                const float g = S.gsig[j] * fexp(rc.q0.w - 0.5f * density_m(rc, v));
                if (fabsf(g) > kMinDensityGrad) N.raw += g, add_outer(N.dA, -0.5f * g, v), N.dens = true;
            }
            if ((S.coloured >> j) & 1u) {
                const float a = fexp(-0.5f * (color_m(rc.q2, rc.q3, v) - S.mmin[j])) * S.inv_a[j];
                if (a >= kMinColourWeight) {
                    const float aw_j = a * S.w[j];
                    aw += aw_j;
                    add_outer(N.cA, -0.5f * aw_j * (gc3 - S.grc[j]), v);
                    N.col = true;
                }
            }
        }
    }
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) N.sh[ch] = N.col && c[ch] > 0.f ? gR[ch] * aw : 0.f;
}

// One pass of gradients over the neighbourhood of site i, each lane adding its own sums with fp32 atomics into its
// neighbour's block: up to 61 atomic instructions per neighbour, each touching one line per lane. With few waves in
// flight (small ray batches) this keeps every lane independent, which is what the latency-bound launch needs.
template <int NV>
__device__ void grad_pass_lane(const MarchField& F, const MarchGradOut& G, int i, bool has, const float (&o)[3],
                               const float (&d)[3], const float (&b)[16], int nb, const float (&gR)[3],
                               const GradBatch& S, float* __restrict__) {
    if (!has) return;
    const int e0 = F.offsets[i], n = F.offsets[i + 1] - e0 + 1;
    for (int e = 0; e < n; ++e) {
        const int k = neighbor(F, i, e0, e);
        NeighbourGrad N;
        neighbour_grad<NV>(F, k, o, d, b, nb, gR, S, N);
        float* gb = G.block + kGradBlock * static_cast<int64_t>(k);
        if (N.dens) {
            unsafeAtomicAdd(gb, N.raw);
#pragma unroll
            for (int u = 0; u < 6; ++u) unsafeAtomicAdd(gb + 1 + u, N.dA[u]);
        }
        if (N.col) {
#pragma unroll
            for (int u = 0; u < 6; ++u) unsafeAtomicAdd(gb + 7 + u, N.cA[u]);
#pragma unroll
            for (int ch = 0; ch < 3; ++ch)
                if (N.sh[ch] != 0.f)
                    for (int jj = 0; jj < nb; ++jj) unsafeAtomicAdd(gb + kGradSh + 3 * jj + ch, b[jj] * N.sh[ch]);
        }
    }
}

// Per lane, a slot of LDS holding the lane's contribution to the current neighbour's gradient block: [0] raw,
// [1..6] density conic, [7..12] colour conic, [13..15] the SH factor gR_c sum_s a_s w_s of each channel, [16..31]
// the lane's SH basis b (set once per ray). 33 floats apart, so that the 64 lanes' slot writes hit distinct banks.
constexpr int kSlot = 33;
constexpr int64_t kCoopRays = 16384;

// The same pass with the atomics shared by the wave. The neighbour loop runs in step across the wave (a lane whose
// pass has fewer neighbours, or none, idles), and at each step the lanes that have a contribution publish it in
// their LDS slot; then the wave adds the rows one at a time, lane t of the wave adding float t of the row's 64-float
// block. A row is one atomic instruction touching two cache lines instead of up to 61 instructions touching 64 lines
// each. With many waves in flight the vector memory pipeline's line rate bounds the per-lane form, and this one wins.
// Adds the rows the lanes of `rows` published in their LDS slots, one row at a time: float t of the 64-float
// gradient block of the row's site k gets slot value t (t < 13) or b_j dc_c (t = 16 + 3 j + c), the wave's active
// lanes taking t = rank, rank + n_act, ... (one atomic instruction per row, two cache lines).
__device__ __forceinline__ void add_rows(const MarchGradOut& G, const float* __restrict__ slots, uint64_t rows, int k,
                                         int nb, int rank, int n_act) {
    while (rows != 0) {
        const int L = __builtin_amdgcn_readfirstlane(__ffsll(static_cast<unsigned long long>(rows)) - 1);
        rows &= rows - 1;
        const int kL = __builtin_amdgcn_readlane(k, L);
        const float* s = slots + kSlot * L;
        float* gb = G.block + kGradBlock * static_cast<int64_t>(kL);
        for (int t = rank; t < kGradBlock; t += n_act) {
            float v = 0.f;
            if (t < 13) {
                v = s[t];
            } else if (t >= kGradSh) {
                const int q = t - kGradSh, j = q / 3;
                if (j < nb) v = s[16 + j] * s[13 + q % 3];
            }
            if (v != 0.f) unsafeAtomicAdd(gb + t, v);
        }
    }
}

template <int NV>
__device__ void grad_pass_wave(const MarchField& F, const MarchGradOut& G, int i, bool has, const float (&o)[3],
                               const float (&d)[3], const float (&b)[16], int nb, const float (&gR)[3],
                               const GradBatch& S, float* __restrict__ slots) {
    const int lane = threadIdx.x & 63;
    int e0 = 0, n = 0;
    if (has) e0 = F.offsets[i], n = F.offsets[i + 1] - e0 + 1;
    float* mine = slots + kSlot * lane;
    const uint64_t act = __ballot(1);
    const int n_act = __popcll(act);
    const int rank = __popcll(act & ((uint64_t(1) << lane) - 1));
    for (int e = 0; __ballot(e < n) != 0; ++e) {
        int k = 0;
        bool row = false;
        if (e < n) {
            k = neighbor(F, i, e0, e);
            NeighbourGrad N;
            neighbour_grad<NV>(F, k, o, d, b, nb, gR, S, N);
            if (N.dens || N.col) {
                mine[0] = N.raw;
#pragma unroll
                for (int u = 0; u < 6; ++u) mine[1 + u] = N.dA[u], mine[7 + u] = N.cA[u];
#pragma unroll
                for (int ch = 0; ch < 3; ++ch) mine[13 + ch] = N.sh[ch];
                row = true;
            }
        }
        __builtin_amdgcn_wave_barrier();
        add_rows(G, slots, __ballot(row), k, nb, rank, n_act);
        __builtin_amdgcn_wave_barrier();
    }
}

// Colour blend of the coloured samples of a pass (flush's sums): A_s and the unnormalised channel sums.
template <int NV>
__device__ void blend_sums(const MarchField& F, int i, const float (&o)[3], const float (&d)[3], const float (&b)[16],
                           int nb, const GradBatch& S, float (&A)[kBatch], float (&cs)[kBatch][3]) {
#pragma unroll
    for (int s = 0; s < kBatch; ++s) A[s] = cs[s][0] = cs[s][1] = cs[s][2] = 0.f;
    const int e0 = F.offsets[i], n = F.offsets[i + 1] - e0 + 1;
    for (int e = 0; e < n; ++e) {
        const int k = neighbor(F, i, e0, e);
        const float4* r = F.rec + block_vec4(NV) * static_cast<int64_t>(k);
        const float4 p = r[0], c0 = r[2], c1 = r[3];
        float c[3];
        sh_eval_n<NV>(r + kRec, b, nb, c);
        c[0] = fmaxf(c[0], 0.f), c[1] = fmaxf(c[1], 0.f), c[2] = fmaxf(c[2], 0.f);
#pragma unroll
        for (int s = 0; s < kBatch; ++s) {
            if (s < S.n && ((S.coloured >> s) & 1u)) {
                float x[3], v[3];
                point_at(o, d, S.t[s], x);
                offset_to(p, x, v);
                const float a = fexp(-0.5f * (color_m(c0, c1, v) - S.mmin[s]));
                A[s] += a, cs[s][0] += a * c[0], cs[s][1] += a * c[1], cs[s][2] += a * c[2];
            }
        }
    }
}

template <int NV, bool COOP>
__device__ void march_ray_backward(const MarchField& F, const MarchParams& M, const MarchRays& R,
                                   const MarchGradIn& GI, const MarchGradOut& G, int64_t r, int cur,
                                   float* __restrict__ slots) {
    const float o[3] = {R.o[3 * r], R.o[3 * r + 1], R.o[3 * r + 2]};
    const float d[3] = {R.d[3 * r], R.d[3 * r + 1], R.d[3 * r + 2]};
    const float near = R.t_near[r], mid = R.t_mid[r], far = R.t_far[r];
    const int n_in = mid > near ? static_cast<int>(ceilf((mid - near) / M.dt)) : 0;
    const int n_total = n_in + M.n_bg;
    const int nb = (F.sh_deg + 1) * (F.sh_deg + 1);
    float b[16];
    sh_basis(d[0], d[1], d[2], F.sh_deg, b);
    const float gR[3] = {GI.g_rgb[3 * r], GI.g_rgb[3 * r + 1], GI.g_rgb[3 * r + 2]};
    const float fg[3] = {GI.rgb[3 * r], GI.rgb[3 * r + 1], GI.rgb[3 * r + 2]};
    const float gT_final = GI.g_T[r] * GI.T[r];
#pragma unroll
    for (int j = 0; j < 16; ++j) slots[kSlot * (threadIdx.x & 63) + 16 + j] = b[j];
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f};
    int k = 0, moves = 0;
    bool live = true;
    while (live && k < n_total) {
        GradBatch S;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            float unused;
            sample_at(near, mid, far, n_in, M, min(k + j, n_total - 1), S.t[j], unused);
        }
        CellPass C;
        cell_pass<block_vec4(NV)>(F, cur, o, d, S.t, C);
        const bool force = moves >= kWalkCap;
        int next = cur;
        bool run = true;
        float Tn[kBatch], delta[kBatch];
        S.n = 0, S.coloured = 0u;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            S.w[j] = S.gsig[j] = S.inv_a[j] = S.grc[j] = Tn[j] = delta[j] = 0.f;
            S.mmin[j] = C.mmin[j];
            if (!run || k + j >= n_total) {
                run = false;
            } else if (C.best[j] == cur || (j == 0 && force)) {
                float t;
                sample_at(near, mid, far, n_in, M, k + j, t, delta[j]);
                const float alpha = 1.f - fexp(-C.sigma[j] * delta[j]);
                const float w = T * alpha;
                ++S.n;
                S.w[j] = w;
                if (w > M.w_thresh) S.coloured |= 1u << j;
                T *= 1.f - alpha;
                Tn[j] = T;
                if (T < M.t_thresh) run = live = false;
            } else {
                next = C.best[j], run = false;
            }
        }
        float A[kBatch], cs[kBatch][3];
        if (S.coloured) blend_sums<NV>(F, cur, o, d, b, nb, S, A, cs);
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            if (j < S.n) {
                float Cj[3] = {0.f, 0.f, 0.f};
                if ((S.coloured >> j) & 1u) {
                    S.inv_a[j] = 1.f / A[j];
#pragma unroll
                    for (int a = 0; a < 3; ++a) Cj[a] = cs[j][a] * S.inv_a[j], acc[a] += S.w[j] * Cj[a];
                    S.grc[j] = gR[0] * Cj[0] + gR[1] * Cj[1] + gR[2] * Cj[2];
                }
                float g = 0.f;
#pragma unroll
                for (int a = 0; a < 3; ++a) g += gR[a] * (Tn[j] * Cj[a] - (fg[a] - acc[a]));
                S.gsig[j] = delta[j] * (g - gT_final);
            }
        }
        if (COOP)
            grad_pass_wave<NV>(F, G, cur, S.n > 0, o, d, b, nb, gR, S, slots);
        else
            grad_pass_lane<NV>(F, G, cur, S.n > 0, o, d, b, nb, gR, S, slots);
        k += S.n;
        moves = S.n > 0 ? 0 : moves;
        if (live && k < n_total && next != cur) cur = next, ++moves;
    }
}

template <bool COOP>
__global__ void __launch_bounds__(kBlock)
    march_backward_kernel(MarchField F, MarchParams M, MarchRays R, MarchGradIn GI, MarchGradOut G) {
    static_assert(kBlock == 64, "the gradient slots are per wave: one wave per workgroup");
    __shared__ float slots[kSlot * 64];
    const int64_t r = xcd_block_id() * kBlock + threadIdx.x;
    if (r >= R.n) return;
    const int cur = R.start[r];
    if (cur < 0 || cur >= F.n_sites) return;  // not traced: no samples, no gradient
    switch (F.sh_deg) {
        case 0: march_ray_backward<sh_vec4_f32(0), COOP>(F, M, R, GI, G, r, cur, slots); break;
        case 1: march_ray_backward<sh_vec4_f32(1), COOP>(F, M, R, GI, G, r, cur, slots); break;
        case 2: march_ray_backward<sh_vec4_f32(2), COOP>(F, M, R, GI, G, r, cur, slots); break;
        default: march_ray_backward<sh_vec4_f32(3), COOP>(F, M, R, GI, G, r, cur, slots); break;
    }
}

// -------------------------------------------------------------------------------------- group layout (small batches)
//
// A training batch of a few thousand rays fills a fraction of the GPU with one ray per lane (4,096 rays are 64
// waves for 1,024 SIMDs), and each ray's samples form a serial chain, so such a launch lasts as long as its slowest
// ray's chain of dependent loads. With kGroup = 16 lanes per ray (4 rays per wave), lane g takes neighbours g,
// g + 16, ... of every neighbourhood, so one round of loads covers a whole neighbourhood (mean 16.5) and the chain
// per sample shrinks from a neighbourhood's length of loads to about one. Per sample: one round at the walk's site
// evaluates the walk's argmin, the density and the colour minimum; the walk moves and repeats the round until its
// site wins or the walk cap is reached (march.cu:157-180); one more round blends a coloured sample's colour (and in
// the backward, one pushes its gradients). Reductions are DPP butterflies inside the 16-lane row: the lexicographic
// (distance, index) minimum, sums and the minimum. Their pairwise operations are commutative, so all lanes of a
// group hold the same bits and composite in step. Sites and walks are those of a sequential scan; the sums differ
// from it by their order of addition (a few ulps).

constexpr int kGroup = 16;

template <int CTRL>
__device__ __forceinline__ void argmin_step(float& d, int& k) {
    const float d2 = row_perm<CTRL>(d);
    const int k2 = row_perm<CTRL>(k);
    if (d2 < d || (d2 == d && k2 < k)) d = d2, k = k2;
}

__device__ __forceinline__ void row_argmin(float& d, int& k) {
    argmin_step<kXor1>(d, k);
    argmin_step<kXor2>(d, k);
    argmin_step<kHalfMirror>(d, k);
    argmin_step<kMirror>(d, k);
}

__device__ __forceinline__ float row_sum(float v) {
    v = v + row_perm<kXor1>(v);
    v = v + row_perm<kXor2>(v);
    v = v + row_perm<kHalfMirror>(v);
    return v + row_perm<kMirror>(v);
}

__device__ __forceinline__ float row_min(float v) {
    v = fminf(v, row_perm<kXor1>(v));
    v = fminf(v, row_perm<kXor2>(v));
    v = fminf(v, row_perm<kHalfMirror>(v));
    return fminf(v, row_perm<kMirror>(v));
}

struct GroupRound {
    float d, sigma, mmin;
    int k;
};

// Walk test, density and colour minimum of point x over the neighbourhood of site i, reduced over the group.
template <int BLK>
__device__ __forceinline__ void group_round(const MarchField& F, int i, const float (&x)[3], int g, GroupRound& Q) {
    const int e0 = F.offsets[i], n = F.offsets[i + 1] - e0 + 1;
    float bd = kInf, s = 0.f, mm = kInf;
    int bk = INT_MAX;
    for (int e = g; e < n; e += kGroup) {
        const int k = neighbor(F, i, e0, e);
        const SiteRec rc = site_rec<BLK>(F, k);
        float v[3];
        offset_to(rc.q0, x, v);
        const float dk = v[0] * v[0] + v[1] * v[1] + v[2] * v[2];
        if (dk < bd || (dk == bd && k < bk)) bd = dk, bk = k;
        s += fexp(rc.q0.w - 0.5f * density_m(rc, v));
        mm = fminf(mm, color_m(rc.q2, rc.q3, v));
    }
    row_argmin(bd, bk);
    Q.d = bd, Q.k = bk, Q.sigma = row_sum(s), Q.mmin = row_min(mm);
}

// The neighbourhood of the group's current cell, as the lanes hold it: lane g's slots are neighbours g and g + 16
// (k = -1 past the end) with their unclamped colours 1/2 + SH_k(d) . b, which depend only on the site and the ray,
// evaluated once per cell visit at its first coloured sample. Neighbours beyond the two slots (cells of more than 32
// neighbours) are read directly at every sample.
constexpr int kSlots = 2;

struct GroupCell {
    int cell, e0, n;
    int k[kSlots];
    float c[kSlots][3];
    bool col_ok;
};

__device__ __forceinline__ void enter_cell(const MarchField& F, int cell, int g, GroupCell& C) {
    C.cell = cell, C.e0 = F.offsets[cell], C.n = F.offsets[cell + 1] - C.e0 + 1, C.col_ok = false;
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
        const int e = g + kGroup * s;
        C.k[s] = e < C.n ? neighbor(F, cell, C.e0, e) : -1;
    }
}

template <int NV>
__device__ __forceinline__ void cell_colours(const MarchField& F, const float (&b)[16], int nb, GroupCell& C) {
    if (C.col_ok) return;
#pragma unroll
    for (int s = 0; s < kSlots; ++s)
        if (C.k[s] >= 0) sh_eval_n<NV>(F.rec + block_vec4(NV) * static_cast<int64_t>(C.k[s]) + kRec, b, nb, C.c[s]);
    C.col_ok = true;
}

// Normalised colour blend at x over the cell's neighbourhood (weights exp(-(m_k - m_min) / 2)): 1 / sum of weights
// and the colour.
template <int NV>
__device__ __forceinline__ void group_colour(const MarchField& F, GroupCell& Cc, const float (&x)[3],
                                             const float (&b)[16], int nb, float mmin, int g, float& inv_a,
                                             float (&C)[3]) {
    cell_colours<NV>(F, b, nb, Cc);
    float A = 0.f, cs[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
        if (Cc.k[s] >= 0) {
            const float4* r = F.rec + block_vec4(NV) * static_cast<int64_t>(Cc.k[s]);
            const float4 p = r[0], c0 = r[2], c1 = r[3];
            float v[3];
            offset_to(p, x, v);
            const float a = fexp(-0.5f * (color_m(c0, c1, v) - mmin));
            A += a;
#pragma unroll
            for (int ch = 0; ch < 3; ++ch) cs[ch] += a * fmaxf(Cc.c[s][ch], 0.f);
        }
    }
    for (int e = g + kGroup * kSlots; e < Cc.n; e += kGroup) {
        const int k = neighbor(F, Cc.cell, Cc.e0, e);
        const float4* r = F.rec + block_vec4(NV) * static_cast<int64_t>(k);
        const float4 p = r[0], c0 = r[2], c1 = r[3];
        float c[3], v[3];
        sh_eval_n<NV>(r + kRec, b, nb, c);
        offset_to(p, x, v);
        const float a = fexp(-0.5f * (color_m(c0, c1, v) - mmin));
        A += a;
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) cs[ch] += a * fmaxf(c[ch], 0.f);
    }
    inv_a = 1.f / row_sum(A);
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) C[ch] = row_sum(cs[ch]) * inv_a;
}

// kGroupBatch consecutive samples per round: one round at the walk's site evaluates, for each of them, the walk's
// argmin, the density and the colour minimum, exactly as a round of its own would (same neighbours per lane in the
// same order, same butterflies), and resolves the leading samples at which the site wins (march_ray's batching in
// the group layout). The coloured samples among them are blended by one colour round. Same bits as one sample per
// round; up to kGroupBatch times fewer rounds.
constexpr int kGroupBatch = 4;

struct GroupRoundN {
    float sigma[kGroupBatch], mmin[kGroupBatch];
    int k[kGroupBatch];
};

template <int BLK>
__device__ __forceinline__ void group_round_n(const MarchField& F, int i, const float (&o)[3], const float (&d)[3],
                                              const float (&t)[kGroupBatch], int g, GroupRoundN& Q) {
    const int e0 = F.offsets[i], n = F.offsets[i + 1] - e0 + 1;
    float bd[kGroupBatch], s[kGroupBatch], mm[kGroupBatch];
    int bk[kGroupBatch];
#pragma unroll
    for (int j = 0; j < kGroupBatch; ++j) bd[j] = kInf, s[j] = 0.f, mm[j] = kInf, bk[j] = INT_MAX;
    for (int e = g; e < n; e += kGroup) {
        const int k = neighbor(F, i, e0, e);
        const SiteRec rc = site_rec<BLK>(F, k);
#pragma unroll
        for (int j = 0; j < kGroupBatch; ++j) {
            float x[3], v[3];
            point_at(o, d, t[j], x);
            offset_to(rc.q0, x, v);
            const float dk = v[0] * v[0] + v[1] * v[1] + v[2] * v[2];
            if (dk < bd[j] || (dk == bd[j] && k < bk[j])) bd[j] = dk, bk[j] = k;
            s[j] += fexp(rc.q0.w - 0.5f * density_m(rc, v));
            mm[j] = fminf(mm[j], color_m(rc.q2, rc.q3, v));
        }
    }
#pragma unroll
    for (int j = 0; j < kGroupBatch; ++j) {
        row_argmin(bd[j], bk[j]);
        Q.k[j] = bk[j], Q.sigma[j] = row_sum(s[j]), Q.mmin[j] = row_min(mm[j]);
    }
}

// group_colour for the coloured samples of one round (bit j of `mask`), each with its own weights and sums.
template <int NV>
__device__ __forceinline__ void group_colour_n(const MarchField& F, GroupCell& Cc, const float (&o)[3],
                                               const float (&d)[3], const float (&t)[kGroupBatch],
                                               const float (&mmin)[kGroupBatch], unsigned mask, const float (&b)[16],
                                               int nb, int g, float (&C)[kGroupBatch][3], float (&inv)[kGroupBatch]) {
    cell_colours<NV>(F, b, nb, Cc);
    float A[kGroupBatch], cs[kGroupBatch][3];
#pragma unroll
    for (int j = 0; j < kGroupBatch; ++j) A[j] = cs[j][0] = cs[j][1] = cs[j][2] = 0.f;
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
        if (Cc.k[s] >= 0) {
            const float4* r = F.rec + block_vec4(NV) * static_cast<int64_t>(Cc.k[s]);
            const float4 p = r[0], c0 = r[2], c1 = r[3];
#pragma unroll
            for (int j = 0; j < kGroupBatch; ++j) {
                if ((mask >> j) & 1u) {
                    float x[3], v[3];
                    point_at(o, d, t[j], x);
                    offset_to(p, x, v);
                    const float a = fexp(-0.5f * (color_m(c0, c1, v) - mmin[j]));
                    A[j] += a;
#pragma unroll
                    for (int ch = 0; ch < 3; ++ch) cs[j][ch] += a * fmaxf(Cc.c[s][ch], 0.f);
                }
            }
        }
    }
    for (int e = g + kGroup * kSlots; e < Cc.n; e += kGroup) {
        const int k = neighbor(F, Cc.cell, Cc.e0, e);
        const float4* r = F.rec + block_vec4(NV) * static_cast<int64_t>(k);
        const float4 p = r[0], c0 = r[2], c1 = r[3];
        float c[3];
        sh_eval_n<NV>(r + kRec, b, nb, c);
#pragma unroll
        for (int j = 0; j < kGroupBatch; ++j) {
            if ((mask >> j) & 1u) {
                float x[3], v[3];
                point_at(o, d, t[j], x);
                offset_to(p, x, v);
                const float a = fexp(-0.5f * (color_m(c0, c1, v) - mmin[j]));
                A[j] += a;
#pragma unroll
                for (int ch = 0; ch < 3; ++ch) cs[j][ch] += a * fmaxf(c[ch], 0.f);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < kGroupBatch; ++j) {
        if ((mask >> j) & 1u) {
            inv[j] = 1.f / row_sum(A[j]);
#pragma unroll
            for (int ch = 0; ch < 3; ++ch) C[j][ch] = row_sum(cs[j][ch]) * inv[j];
        }
    }
}

// Per ray: the sample loop of march_ray, kGroupBatch samples per round.
template <int NV, bool TRACE>
__device__ void march_ray_group(const MarchField& F, const MarchParams& M, const MarchRays& R, const MarchOut& O,
                                int64_t r, int cur, int g) {
    const float o[3] = {R.o[3 * r], R.o[3 * r + 1], R.o[3 * r + 2]};
    const float d[3] = {R.d[3 * r], R.d[3 * r + 1], R.d[3 * r + 2]};
    const float near = R.t_near[r], mid = R.t_mid[r], far = R.t_far[r];
    const int n_in = mid > near ? static_cast<int>(ceilf((mid - near) / M.dt)) : 0;
    const int n_total = n_in + M.n_bg;
    const int nb = (F.sh_deg + 1) * (F.sh_deg + 1);
    float b[16];
    sh_basis(d[0], d[1], d[2], F.sh_deg, b);
    int n_samples = 0, n_color = 0, walk_steps = 0, moves = 0;
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f}, dep = 0.f;
    GroupCell Cc;
    Cc.cell = -1;
    bool live = true;
    for (int k = 0; live && k < n_total;) {
        float t[kGroupBatch], delta[kGroupBatch], w[kGroupBatch];
#pragma unroll
        for (int j = 0; j < kGroupBatch; ++j)
            sample_at(near, mid, far, n_in, M, min(k + j, n_total - 1), t[j], delta[j]);
        GroupRoundN Q;
        group_round_n<block_vec4(NV)>(F, cur, o, d, t, g, Q);
        int nres = 0, next = cur;
        unsigned coloured = 0u;
        bool run = true;
#pragma unroll
        for (int j = 0; j < kGroupBatch; ++j) {
            w[j] = 0.f;
            if (!run || k + j >= n_total) {
                run = false;
            } else if (Q.k[j] == cur || (j == 0 && moves >= kWalkCap)) {
                if (TRACE && g == 0 && n_samples < O.trace_cap) O.trace[r * O.trace_cap + n_samples] = cur;
                const float alpha = 1.f - fexp(-Q.sigma[j] * delta[j]);
                w[j] = T * alpha;
                ++n_samples, ++nres;
                if (w[j] > M.w_thresh) coloured |= 1u << j, ++n_color;
                T *= 1.f - alpha;
                if (T < M.t_thresh) run = live = false;
            } else {
                next = Q.k[j], run = false;
            }
        }
        if (coloured) {
            if (Cc.cell != cur) enter_cell(F, cur, g, Cc);
            float C[kGroupBatch][3], inv[kGroupBatch];
            group_colour_n<NV>(F, Cc, o, d, t, Q.mmin, coloured, b, nb, g, C, inv);
#pragma unroll
            for (int j = 0; j < kGroupBatch; ++j) {
                if ((coloured >> j) & 1u) {
#pragma unroll
                    for (int a = 0; a < 3; ++a) acc[a] += w[j] * C[j][a];
                    dep += w[j] * t[j];
                }
            }
        }
        k += nres;
        moves = nres > 0 ? 0 : moves;
        if (live && k < n_total && next != cur) cur = next, ++walk_steps, ++moves;
    }
    if (g == 0) {
#pragma unroll
        for (int a = 0; a < 3; ++a) O.rgb[3 * r + a] = acc[a];
        O.T[r] = T;
        O.depth[r] = dep;
        O.stats[3 * r] = n_samples, O.stats[3 * r + 1] = n_color, O.stats[3 * r + 2] = walk_steps;
    }
}

template <bool TRACE>
__global__ void __launch_bounds__(kBlock) march_group_kernel(MarchField F, MarchParams M, MarchRays R, MarchOut O) {
    const int64_t i = (xcd_block_id() * kBlock + threadIdx.x) / kGroup;
    const int g = threadIdx.x % kGroup;
    if (i >= R.n) return;
    const int64_t r = R.order != nullptr ? R.order[i] : i;
    if (r < 0 || r >= R.n) return;  // not a permutation entry: the whole group leaves
    const int cur = R.start[r];
    if (cur < 0 || cur >= F.n_sites) {  // not traced: empty foreground
        if (g == 0) {
            O.rgb[3 * r] = O.rgb[3 * r + 1] = O.rgb[3 * r + 2] = 0.f;
            O.T[r] = 1.f, O.depth[r] = 0.f;
            O.stats[3 * r] = O.stats[3 * r + 1] = O.stats[3 * r + 2] = 0;
        }
        return;
    }
    switch (F.sh_deg) {
        case 0: march_ray_group<sh_vec4_f32(0), TRACE>(F, M, R, O, r, cur, g); break;
        case 1: march_ray_group<sh_vec4_f32(1), TRACE>(F, M, R, O, r, cur, g); break;
        case 2: march_ray_group<sh_vec4_f32(2), TRACE>(F, M, R, O, r, cur, g); break;
        default: march_ray_group<sh_vec4_f32(3), TRACE>(F, M, R, O, r, cur, g); break;
    }
}

// A slot's gradient sums over the samples of one cell visit: raw, the density conic, the colour conic and
// sum_s a_s w_s (the SH gradient is b_j gR_c times it, for the channels whose unclamped colour is positive).
struct SlotGrad {
    float raw, dA[6], cA[6], aw;
    bool dens, col;
};

__device__ __forceinline__ void clear_slot(SlotGrad& A) {
    A.raw = A.aw = 0.f;
#pragma unroll
    for (int u = 0; u < 6; ++u) A.dA[u] = A.cA[u] = 0.f;
    A.dens = A.col = false;
}

// One sample's contribution to neighbour k (record rc) at x, with the neighbour's unclamped colour c.
__device__ __forceinline__ void sample_grad(const SiteRec& rc, const float (&x)[3], const float (&c)[3],
                                            const float (&gR)[3], float gsig, bool coloured, float w, float mmin,
                                            float inv_a, float grc, SlotGrad& A) {
    float v[3];
    offset_to(rc.q0, x, v);
    if (gsig != 0.f) {
        const float gd = gsig * fexp(rc.q0.w - 0.5f * density_m(rc, v));
        if (fabsf(gd) > kMinDensityGrad) A.raw += gd, add_outer(A.dA, -0.5f * gd, v), A.dens = true;
    }
    if (coloured) {
        const float a = fexp(-0.5f * (color_m(rc.q2, rc.q3, v) - mmin)) * inv_a;
        if (a >= kMinColourWeight) {
            const float aw = a * w;
            const float gc3 = gR[0] * fmaxf(c[0], 0.f) + gR[1] * fmaxf(c[1], 0.f) + gR[2] * fmaxf(c[2], 0.f);
            A.aw += aw;
            add_outer(A.cA, -0.5f * aw * (gc3 - grc), v);
            A.col = true;
        }
    }
}

__device__ __forceinline__ void flush_slot(const MarchGradOut& G, int k, const float (&c)[3], const float (&b)[16],
                                           int nb, const float (&gR)[3], const SlotGrad& A) {
    float* gb = G.block + kGradBlock * static_cast<int64_t>(k);
    if (A.dens) {
        unsafeAtomicAdd(gb, A.raw);
#pragma unroll
        for (int u = 0; u < 6; ++u) unsafeAtomicAdd(gb + 1 + u, A.dA[u]);
    }
    if (A.col) {
#pragma unroll
        for (int u = 0; u < 6; ++u) unsafeAtomicAdd(gb + 7 + u, A.cA[u]);
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) {
            const float dc = c[ch] > 0.f ? gR[ch] * A.aw : 0.f;
            if (dc != 0.f)
                for (int jj = 0; jj < nb; ++jj) unsafeAtomicAdd(gb + kGradSh + 3 * jj + ch, b[jj] * dc);
        }
    }
}

// The backward of march_ray_group: the same rounds replay the same samples bit for bit. Each lane sums its slots'
// gradients over the samples of a cell visit in registers and adds them with atomics when the ray leaves the cell
// (or ends), so a visit of several samples costs one set of atomics per neighbour; neighbours beyond the slots add
// theirs per sample. The formulas are those of march_ray_backward.
template <int NV>
__device__ void march_ray_group_backward(const MarchField& F, const MarchParams& M, const MarchRays& R,
                                         const MarchGradIn& GI, const MarchGradOut& G, int64_t r, int cur, int g,
                                         float* __restrict__ slots) {
    const float o[3] = {R.o[3 * r], R.o[3 * r + 1], R.o[3 * r + 2]};
    const float d[3] = {R.d[3 * r], R.d[3 * r + 1], R.d[3 * r + 2]};
    const float near = R.t_near[r], mid = R.t_mid[r], far = R.t_far[r];
    const int n_in = mid > near ? static_cast<int>(ceilf((mid - near) / M.dt)) : 0;
    const int n_total = n_in + M.n_bg;
    const int nb = (F.sh_deg + 1) * (F.sh_deg + 1);
    float b[16];
    sh_basis(d[0], d[1], d[2], F.sh_deg, b);
    const float gR[3] = {GI.g_rgb[3 * r], GI.g_rgb[3 * r + 1], GI.g_rgb[3 * r + 2]};
    const float fg[3] = {GI.rgb[3 * r], GI.rgb[3 * r + 1], GI.rgb[3 * r + 2]};
    const float gT_final = GI.g_T[r] * GI.T[r];
#pragma unroll
    for (int j = 0; j < 16; ++j) slots[kSlot * (threadIdx.x & 63) + 16 + j] = b[j];
    int moves = 0;
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f};
    GroupCell Cc;
    Cc.cell = -1;
    SlotGrad S[kSlots];
#pragma unroll
    for (int s = 0; s < kSlots; ++s) clear_slot(S[s]);
    // the slots' sums of the visit just left, added as rows shared by the resolving lanes of the wave
    auto flush = [&]() {
        if (Cc.cell < 0) return;
        const int lane = threadIdx.x & 63;
        float* mine = slots + kSlot * lane;
        const uint64_t act = __ballot(1);
        const int n_act = __popcll(act);
        const int rank = __popcll(act & ((uint64_t(1) << lane) - 1));
#pragma unroll
        for (int s = 0; s < kSlots; ++s) {
            const bool row = Cc.k[s] >= 0 && (S[s].dens || S[s].col);
            if (row) {
                mine[0] = S[s].raw;
#pragma unroll
                for (int u = 0; u < 6; ++u) mine[1 + u] = S[s].dA[u], mine[7 + u] = S[s].cA[u];
#pragma unroll
                for (int ch = 0; ch < 3; ++ch) mine[13 + ch] = S[s].col && Cc.c[s][ch] > 0.f ? gR[ch] * S[s].aw : 0.f;
            }
            __builtin_amdgcn_wave_barrier();
            add_rows(G, slots, __ballot(row), Cc.k[s], nb, rank, n_act);
            __builtin_amdgcn_wave_barrier();
            clear_slot(S[s]);
        }
    };
    for (int k = 0; k < n_total;) {
        float t, delta, x[3];
        sample_at(near, mid, far, n_in, M, k, t, delta);
        point_at(o, d, t, x);
        GroupRound Q;
        group_round<block_vec4(NV)>(F, cur, x, g, Q);
        if (Q.k != cur && moves < kWalkCap) {
            cur = Q.k, ++moves;
            continue;
        }
        moves = 0;
        if (Cc.cell != cur) flush(), enter_cell(F, cur, g, Cc);
        const float alpha = 1.f - fexp(-Q.sigma * delta);
        const float w = T * alpha;
        const float T_next = T * (1.f - alpha);
        const bool coloured = w > M.w_thresh;
        float inv_a = 0.f, C[3] = {0.f, 0.f, 0.f}, grc = 0.f;
        if (coloured) {
            group_colour<NV>(F, Cc, x, b, nb, Q.mmin, g, inv_a, C);
#pragma unroll
            for (int a = 0; a < 3; ++a) acc[a] += w * C[a];
            grc = gR[0] * C[0] + gR[1] * C[1] + gR[2] * C[2];
        }
        float gs = 0.f;
#pragma unroll
        for (int a = 0; a < 3; ++a) gs += gR[a] * (T_next * C[a] - (fg[a] - acc[a]));
        const float gsig = delta * (gs - gT_final);
#pragma unroll
        for (int s = 0; s < kSlots; ++s) {
            if (Cc.k[s] >= 0) {
                const SiteRec rc = site_rec<block_vec4(NV)>(F, Cc.k[s]);
                const float c[3] = {Cc.col_ok ? Cc.c[s][0] : 0.f, Cc.col_ok ? Cc.c[s][1] : 0.f,
                                    Cc.col_ok ? Cc.c[s][2] : 0.f};
                sample_grad(rc, x, c, gR, gsig, coloured, w, Q.mmin, inv_a, grc, S[s]);
            }
        }
        for (int e = g + kGroup * kSlots; e < Cc.n; e += kGroup) {
            const int kk = neighbor(F, cur, Cc.e0, e);
            const float4* rp = F.rec + block_vec4(NV) * static_cast<int64_t>(kk);
            const SiteRec rc = {rp[0], rp[1], rp[2], rp[3]};
            float c[3] = {0.f, 0.f, 0.f};
            if (coloured) sh_eval_n<NV>(rp + kRec, b, nb, c);
            SlotGrad A;
            clear_slot(A);
            sample_grad(rc, x, c, gR, gsig, coloured, w, Q.mmin, inv_a, grc, A);
            flush_slot(G, kk, c, b, nb, gR, A);
        }
        T = T_next;
        ++k;
        if (T < M.t_thresh) break;
    }
    flush();
}

__global__ void __launch_bounds__(kBlock)
    march_group_backward_kernel(MarchField F, MarchParams M, MarchRays R, MarchGradIn GI, MarchGradOut G) {
    static_assert(kBlock == 64, "the gradient slots are per wave: one wave per workgroup");
    __shared__ float slots[kSlot * 64];
    const int64_t r = (xcd_block_id() * kBlock + threadIdx.x) / kGroup;
    const int g = threadIdx.x % kGroup;
    if (r >= R.n) return;
    const int cur = R.start[r];
    if (cur < 0 || cur >= F.n_sites) return;
    switch (F.sh_deg) {
        case 0: march_ray_group_backward<sh_vec4_f32(0)>(F, M, R, GI, G, r, cur, g, slots); break;
        case 1: march_ray_group_backward<sh_vec4_f32(1)>(F, M, R, GI, G, r, cur, g, slots); break;
        case 2: march_ray_group_backward<sh_vec4_f32(2)>(F, M, R, GI, G, r, cur, g, slots); break;
        default: march_ray_group_backward<sh_vec4_f32(3)>(F, M, R, GI, G, r, cur, g, slots); break;
    }
}

// ---------------------------------------------------------------------- training renderer (foam.cu), 16 lanes per ray
//
// The samples of foam.cu:1-17: x(near) in the cell the walk reaches, then every crossing of a Voronoi face (the
// nearest bisector plane ahead of the ray, ties to the smaller neighbour index), then x(far); trapezoid compositing
// of consecutive samples, colours only for segments of weight > w_thresh. Same group layout and site blocks as the
// 16-lane march. A crossing sample's site is the cell the ray enters, whose neighbourhood is also the one that gives
// that cell's exit, so one round over it evaluates the sample's density and colour minimum and the cell's exit
// candidates together: one round per sample, plus one colour round for a sample of a coloured segment. The forward
// can record every sample (t, site, sigma, C, m_min, 1 / A or 0: foam.cu:272-286) for the backward, which replays
// the records or re-traces rays that did not fit with the same rounds (same bits).

constexpr int kTrainRecord = 8;

struct TrainSample {
    float t, sigma, mmin, inv_a, C[3];
    int site;
    bool has_c;
};

// Density and colour minimum at x over the neighbourhood of i, and the exit of cell i along the ray (smallest
// bisector parameter ahead, ties to the smaller index; INT_MAX when none), reduced over the group.
template <int BLK>
__device__ __forceinline__ void train_round(const MarchField& F, int i, const float (&o)[3], const float (&d)[3],
                                            float t, int g, TrainSample& S, float& t_exit, int& next) {
    float x[3];
    point_at(o, d, t, x);
    const int e0 = F.offsets[i], n = F.offsets[i + 1] - e0 + 1;
    const float4 pi = F.rec[BLK * static_cast<int64_t>(i)];
    float s = 0.f, mm = kInf, bt = kInf;
    int bk = INT_MAX;
    for (int e = g; e < n; e += kGroup) {
        const int k = neighbor(F, i, e0, e);
        const SiteRec rc = site_rec<BLK>(F, k);
        float v[3];
        offset_to(rc.q0, x, v);
        s += fexp(rc.q0.w - 0.5f * density_m(rc, v));
        mm = fminf(mm, color_m(rc.q2, rc.q3, v));
        if (e > 0) {
            const float nn[3] = {rc.q0.x - pi.x, rc.q0.y - pi.y, rc.q0.z - pi.z};
            const float m[3] = {0.5f * (rc.q0.x + pi.x) - o[0], 0.5f * (rc.q0.y + pi.y) - o[1],
                                0.5f * (rc.q0.z + pi.z) - o[2]};
            const float dn = nn[0] * d[0] + nn[1] * d[1] + nn[2] * d[2];
            if (dn > 0.f) {
                const float tj = (m[0] * nn[0] + m[1] * nn[1] + m[2] * nn[2]) / dn;
                if (tj < bt || (tj == bt && k < bk)) bt = tj, bk = k;
            }
        }
    }
    row_argmin(bt, bk);
    S.t = t, S.site = i, S.sigma = row_sum(s), S.mmin = row_min(mm), S.has_c = false, S.inv_a = 0.f;
    S.C[0] = S.C[1] = S.C[2] = 0.f;
    t_exit = bt, next = bk;
}

// Normalised colour blend of sample S (weights exp(-(m_k - m_min) / 2) over its site's neighbourhood).
template <int NV>
__device__ __forceinline__ void train_colour(const MarchField& F, const float (&o)[3], const float (&d)[3],
                                             const float (&b)[16], int nb, int g, TrainSample& S) {
    float x[3];
    point_at(o, d, S.t, x);
    const int e0 = F.offsets[S.site], n = F.offsets[S.site + 1] - e0 + 1;
    float A = 0.f, cs[3] = {0.f, 0.f, 0.f};
    for (int e = g; e < n; e += kGroup) {
        const int k = neighbor(F, S.site, e0, e);
        const float4* r = F.rec + block_vec4(NV) * static_cast<int64_t>(k);
        const float4 p = r[0], c0 = r[2], c1 = r[3];
        float c[3], v[3];
        sh_eval_n<NV>(r + kRec, b, nb, c);
        offset_to(p, x, v);
        const float a = fexp(-0.5f * (color_m(c0, c1, v) - S.mmin));
        A += a;
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) cs[ch] += a * fmaxf(c[ch], 0.f);
    }
    S.inv_a = 1.f / row_sum(A);
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) S.C[ch] = row_sum(cs[ch]) * S.inv_a;
    S.has_c = true;
}

// Greedy walk of the group from `cur` to the site nearest x(t) (march.cu / foam.cu walk_to).
template <int BLK>
__device__ __forceinline__ int train_walk(const MarchField& F, int cur, const float (&o)[3], const float (&d)[3],
                                          float t, int g, int& steps) {
    float x[3];
    point_at(o, d, t, x);
    for (int it = 0; it < kWalkCap; ++it) {
        GroupRound Q;
        group_round<BLK>(F, cur, x, g, Q);
        if (Q.k == cur) break;
        cur = Q.k, ++steps;
    }
    return cur;
}

__device__ __forceinline__ void train_store(float* __restrict__ rec, int64_t r, int K, int s, const TrainSample& S,
                                            int g) {
    if (rec == nullptr || s >= K || g >= kTrainRecord) return;
    const float v = g == 0 ? S.t
                  : g == 1 ? __int_as_float(S.site)
                  : g == 2 ? S.sigma
                  : g == 3 ? S.C[0]
                  : g == 4 ? S.C[1]
                  : g == 5 ? S.C[2]
                  : g == 6 ? S.mmin
                           : (S.has_c ? S.inv_a : 0.f);
    rec[(r * K + s) * kTrainRecord + g] = v;
}

__device__ __forceinline__ void train_load(const float* __restrict__ rec, int64_t r, int K, int s, TrainSample& S) {
    const float* p = rec + (r * K + s) * kTrainRecord;
    S.t = p[0], S.site = __float_as_int(p[1]), S.sigma = p[2];
    S.C[0] = p[3], S.C[1] = p[4], S.C[2] = p[5];
    S.mmin = p[6], S.inv_a = p[7], S.has_c = p[7] > 0.f;
}

struct TrainRays {
    const float* __restrict__ o;
    const float* __restrict__ d;
    const int* __restrict__ start;
    const float* __restrict__ t_near;
    const float* __restrict__ t_far;
    int64_t n;
};

template <int NV>
__device__ void train_ray(const MarchField& F, const MarchParams& M, const TrainRays& R, const MarchOut& O,
                          float* __restrict__ rec, int K, int64_t r, int g) {
    const float o[3] = {R.o[3 * r], R.o[3 * r + 1], R.o[3 * r + 2]};
    const float d[3] = {R.d[3 * r], R.d[3 * r + 1], R.d[3 * r + 2]};
    const float near = R.t_near[r], far = R.t_far[r];
    const int nb = (F.sh_deg + 1) * (F.sh_deg + 1);
    float b[16];
    sh_basis(d[0], d[1], d[2], F.sh_deg, b);
    int walk_steps = 0, n_samples = 1, n_color = 0;
    int cur = train_walk<block_vec4(NV)>(F, R.start[r], o, d, near, g, walk_steps);
    TrainSample P, Q;
    float te, te2;
    int nx, nx2;
    train_round<block_vec4(NV)>(F, cur, o, d, near, g, P, te, nx);
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f}, dep = 0.f;
    for (int it = 0; it < kMaxCells; ++it) {
        const bool last = nx == INT_MAX || te >= far;
        train_round<block_vec4(NV)>(F, last ? cur : nx, o, d, last ? far : fmaxf(te, P.t), g, Q, te2, nx2);
        ++n_samples;
        const float delta = Q.t - P.t;
        const float alpha = 1.f - fexp(-0.5f * (P.sigma + Q.sigma) * delta);
        const float w = T * alpha;
        if (w > M.w_thresh) {
            if (!P.has_c) train_colour<NV>(F, o, d, b, nb, g, P);
            train_colour<NV>(F, o, d, b, nb, g, Q);
#pragma unroll
            for (int a = 0; a < 3; ++a) acc[a] += w * 0.5f * (P.C[a] + Q.C[a]);
            dep += w * 0.5f * (P.t + Q.t);
            ++n_color;
        }
        T *= 1.f - alpha;
        train_store(rec, r, K, n_samples - 2, P, g);
        P = Q;
        cur = Q.site, te = te2, nx = nx2;
        if (last || T < M.t_thresh) break;
    }
    train_store(rec, r, K, n_samples - 1, P, g);
    if (g == 0) {
#pragma unroll
        for (int a = 0; a < 3; ++a) O.rgb[3 * r + a] = acc[a];
        O.T[r] = T;
        O.depth[r] = dep;
        O.stats[3 * r] = n_samples, O.stats[3 * r + 1] = n_color, O.stats[3 * r + 2] = walk_steps;
    }
}

__global__ void __launch_bounds__(kBlock)
    train_forward_kernel(MarchField F, MarchParams M, TrainRays R, MarchOut O, float* __restrict__ rec, int K) {
    const int64_t r = (xcd_block_id() * kBlock + threadIdx.x) / kGroup;
    const int g = threadIdx.x % kGroup;
    if (r >= R.n) return;
    const int cur = R.start[r];
    if (cur < 0 || cur >= F.n_sites) {  // not traced: empty foreground, no samples
        if (g == 0) {
            O.rgb[3 * r] = O.rgb[3 * r + 1] = O.rgb[3 * r + 2] = 0.f;
            O.T[r] = 1.f, O.depth[r] = 0.f;
            O.stats[3 * r] = O.stats[3 * r + 1] = O.stats[3 * r + 2] = 0;
        }
        return;
    }
    switch (F.sh_deg) {
        case 0: train_ray<sh_vec4_f32(0)>(F, M, R, O, rec, K, r, g); break;
        case 1: train_ray<sh_vec4_f32(1)>(F, M, R, O, rec, K, r, g); break;
        case 2: train_ray<sh_vec4_f32(2)>(F, M, R, O, rec, K, r, g); break;
        default: train_ray<sh_vec4_f32(3)>(F, M, R, O, rec, K, r, g); break;
    }
}

// A sample's gradients (gs = dL/dsigma, gC = dL/dC) over its site's neighbourhood (foam.cu:303-343). Each lane
// computes its neighbours' contributions and publishes them in its LDS slot; the wave adds the rows with add_rows
// (scattered fp32 atomics, one per lane and float, ran this kernel at ~16 G atomics/s, where a row is one atomic
// instruction on two lines). The neighbour rounds run in step across the wave: every active lane takes part in
// every round, lanes of rays with fewer neighbours (or nothing to add) idle.
template <int NV>
__device__ void train_scatter(const MarchField& F, const MarchGradOut& G, const float (&o)[3], const float (&d)[3],
                              const float (&b)[16], int nb, const TrainSample& S, float gs, const float (&gC)[3],
                              int g, float* __restrict__ slots) {
    const bool colour = S.has_c && (gC[0] != 0.f || gC[1] != 0.f || gC[2] != 0.f);
    int e0 = 0, n = 0;
    if (gs != 0.f || colour) e0 = F.offsets[S.site], n = F.offsets[S.site + 1] - e0 + 1;
    float x[3];
    point_at(o, d, S.t, x);
    const float gCC = gC[0] * S.C[0] + gC[1] * S.C[1] + gC[2] * S.C[2];
    const int lane = threadIdx.x & 63;
    float* mine = slots + kSlot * lane;
    const uint64_t act = __ballot(1);
    const int n_act = __popcll(act);
    const int rank = __popcll(act & ((uint64_t(1) << lane) - 1));
    for (int base = 0; __ballot(base < n) != 0; base += kGroup) {
        const int e = base + g;
        int k = 0;
        bool row = false;
        if (e < n) {
            k = neighbor(F, S.site, e0, e);
            const float4* rp = F.rec + block_vec4(NV) * static_cast<int64_t>(k);
            const SiteRec rc = {rp[0], rp[1], rp[2], rp[3]};
            float v[3];
            offset_to(rc.q0, x, v);
            float graw = 0.f, gdA[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, gcA[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            float dc[3] = {0.f, 0.f, 0.f};
            if (gs != 0.f) {
                const float gd = gs * fexp(rc.q0.w - 0.5f * density_m(rc, v));
                if (fabsf(gd) > kMinDensityGrad) graw = gd, add_outer(gdA, -0.5f * gd, v), row = true;
            }
            if (colour) {
                const float a = fexp(-0.5f * (color_m(rc.q2, rc.q3, v) - S.mmin)) * S.inv_a;
                if (a >= kMinColourWeight) {
                    float c[3];
                    sh_eval_n<NV>(rp + kRec, b, nb, c);
#pragma unroll
                    for (int ch = 0; ch < 3; ++ch) dc[ch] = c[ch] > 0.f ? a * gC[ch] : 0.f;
                    const float ga = gC[0] * fmaxf(c[0], 0.f) + gC[1] * fmaxf(c[1], 0.f) + gC[2] * fmaxf(c[2], 0.f);
                    const float gm = -0.5f * a * (ga - gCC);
                    if (gm != 0.f) add_outer(gcA, gm, v);
                    row = true;
                }
            }
            if (row) {
                mine[0] = graw;
#pragma unroll
                for (int u = 0; u < 6; ++u) mine[1 + u] = gdA[u], mine[7 + u] = gcA[u];
#pragma unroll
                for (int ch = 0; ch < 3; ++ch) mine[13 + ch] = dc[ch];
            }
        }
        __builtin_amdgcn_wave_barrier();
        add_rows(G, slots, __ballot(row), k, nb, rank, n_act);
        __builtin_amdgcn_wave_barrier();
    }
}

// foam.cu:395-469: every sample collects half of the gradients of the segments on both sides.
template <int NV>
__device__ void train_ray_backward(const MarchField& F, const MarchParams& M, const TrainRays& R,
                                   const MarchGradIn& GI, const MarchGradOut& G, const float* __restrict__ rec, int K,
                                   const int* __restrict__ stats, int64_t r, int g, float* __restrict__ slots) {
    const float o[3] = {R.o[3 * r], R.o[3 * r + 1], R.o[3 * r + 2]};
    const float d[3] = {R.d[3 * r], R.d[3 * r + 1], R.d[3 * r + 2]};
    const float near = R.t_near[r], far = R.t_far[r];
    const int nb = (F.sh_deg + 1) * (F.sh_deg + 1);
    float b[16];
    sh_basis(d[0], d[1], d[2], F.sh_deg, b);
    const float gR[3] = {GI.g_rgb[3 * r], GI.g_rgb[3 * r + 1], GI.g_rgb[3 * r + 2]};
    const float fg[3] = {GI.rgb[3 * r], GI.rgb[3 * r + 1], GI.rgb[3 * r + 2]};
    const float gT_final = GI.g_T[r] * GI.T[r];
#pragma unroll
    for (int j = 0; j < 16; ++j) slots[kSlot * (threadIdx.x & 63) + 16 + j] = b[j];
    const int n_stored = rec != nullptr && stats[3 * r] <= K ? stats[3 * r] : 0;
    TrainSample P, Q;
    float te = 0.f, te2 = 0.f;
    int nx = INT_MAX, nx2 = INT_MAX, cur = 0;
    if (n_stored > 0) {
        train_load(rec, r, K, 0, P);
    } else {
        int steps = 0;
        cur = train_walk<block_vec4(NV)>(F, R.start[r], o, d, near, g, steps);
        train_round<block_vec4(NV)>(F, cur, o, d, near, g, P, te, nx);
    }
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f}, gs_pending = 0.f, gC_pending[3] = {0.f, 0.f, 0.f};
    for (int it = 0; it < kMaxCells; ++it) {
        bool last;
        if (n_stored > 0) {
            if (it + 1 >= n_stored) break;
            train_load(rec, r, K, it + 1, Q);
            last = it + 2 >= n_stored;
        } else {
            last = nx == INT_MAX || te >= far;
            train_round<block_vec4(NV)>(F, last ? cur : nx, o, d, last ? far : fmaxf(te, P.t), g, Q, te2, nx2);
        }
        const float delta = Q.t - P.t;
        const float alpha = 1.f - fexp(-0.5f * (P.sigma + Q.sigma) * delta);
        const float w = T * alpha;
        const float T_next = T * (1.f - alpha);
        const bool active = w > M.w_thresh;
        float c[3] = {0.f, 0.f, 0.f};
        if (active) {
            if (!P.has_c) train_colour<NV>(F, o, d, b, nb, g, P);
            if (!Q.has_c) train_colour<NV>(F, o, d, b, nb, g, Q);
#pragma unroll
            for (int a = 0; a < 3; ++a) c[a] = 0.5f * (P.C[a] + Q.C[a]), acc[a] += w * c[a];
        }
        float g_sbar = 0.f;
#pragma unroll
        for (int a = 0; a < 3; ++a) g_sbar += gR[a] * (T_next * c[a] - (fg[a] - acc[a]));
        g_sbar = delta * (g_sbar - gT_final);
        float gc_half[3], gC_P[3];
#pragma unroll
        for (int a = 0; a < 3; ++a) gc_half[a] = active ? 0.5f * w * gR[a] : 0.f, gC_P[a] = gC_pending[a] + gc_half[a];
        train_scatter<NV>(F, G, o, d, b, nb, P, gs_pending + 0.5f * g_sbar, gC_P, g, slots);
        gs_pending = 0.5f * g_sbar;
#pragma unroll
        for (int a = 0; a < 3; ++a) gC_pending[a] = gc_half[a];
        T = T_next;
        P = Q;
        cur = Q.site, te = te2, nx = nx2;
        if (last || T < M.t_thresh) break;
    }
    train_scatter<NV>(F, G, o, d, b, nb, P, gs_pending, gC_pending, g, slots);
}

__global__ void __launch_bounds__(kBlock)
    train_backward_kernel(MarchField F, MarchParams M, TrainRays R, MarchGradIn GI, MarchGradOut G,
                          const float* __restrict__ rec, int K, const int* __restrict__ stats) {
    static_assert(kBlock == 64, "the gradient slots are per wave: one wave per workgroup");
    __shared__ float slots[kSlot * 64];
    const int64_t r = (xcd_block_id() * kBlock + threadIdx.x) / kGroup;
    const int g = threadIdx.x % kGroup;
    if (r >= R.n) return;
    if (R.start[r] < 0 || R.start[r] >= F.n_sites) return;  // not traced: no gradient
    switch (F.sh_deg) {
        case 0: train_ray_backward<sh_vec4_f32(0)>(F, M, R, GI, G, rec, K, stats, r, g, slots); break;
        case 1: train_ray_backward<sh_vec4_f32(1)>(F, M, R, GI, G, rec, K, stats, r, g, slots); break;
        case 2: train_ray_backward<sh_vec4_f32(2)>(F, M, R, GI, G, rec, K, stats, r, g, slots); break;
        default: train_ray_backward<sh_vec4_f32(3)>(F, M, R, GI, G, rec, K, stats, r, g, slots); break;
    }
}

// Grid-stride fill with zeros (a kernel, not a memset, so that a captured stream records no memset node).
constexpr int64_t kZeroBlocks = 4096;
__global__ void __launch_bounds__(256) zero_kernel(float* __restrict__ p, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += kZeroBlocks * 256) p[i] = 0.f;
}

}  // namespace
}  // namespace vgr

extern "C" int64_t vgr_march_work_size(int64_t n_sites, int64_t sh_deg) {
    using namespace vgr;
    if (n_sites <= 0 || sh_deg < 0 || sh_deg > 3) return 0;
    return n_sites * static_cast<int64_t>(sizeof(float4)) * block_vec4(sh_vec4_f32(static_cast<int>(sh_deg)));
}

extern "C" int64_t vgr_march_backward_work_size(int64_t n_sites, int64_t sh_deg) {
    const int64_t fwd = vgr_march_work_size(n_sites, sh_deg);
    return fwd > 0 ? fwd + n_sites * static_cast<int64_t>(sizeof(float)) * vgr::kGradBlock : 0;
}

namespace vgr {
namespace {
// Launches of fewer rays take the 16-lane group layout, for forward and backward alike (the backward replays the
// forward's sums). Config 5, ms forward / backward, one ray per lane against 16 lanes per ray: 4,096 rays 34 / 85
// against 5 / 16; 65,536 rays 41 / 189 against 19 / 70; 262,144 rays 75 / 408 against 67 / 251; 1,048,576 rays
// 236 / 1531 against 255 / 974. A training step (forward + backward) is faster in the group layout at every size
// measured, a forward alone from about half a million rays in one ray per lane (the whole 16.7M-ray inference
// batch: 3,350 against 5,264 ms), hence the switch at 2^19 rays.
constexpr int64_t kGroupRays = 524288;

int64_t march_lanes(int64_t lanes, int64_t n_rays) { return lanes != 0 ? lanes : n_rays < kGroupRays ? kGroup : 1; }
}  // namespace
}  // namespace vgr

extern "C" int vgr_march_forward_lanes(const float* points, int64_t n_sites, const int32_t* offsets,
                                       const int32_t* adj, int64_t n_adj, const float* raw, const float* dA,
                                       const float* cA, const float* sh, int64_t sh_deg, const float* o,
                                       const float* d, const int32_t* start, const float* near_t,
                                       const float* mid_t, const float* far_t, int64_t n_rays, double dt,
                                       int64_t n_bg, double t_thresh, double w_thresh, float* rgb, float* T,
                                       float* depth, int32_t* stats, int32_t* trace, int64_t trace_cap,
                                       const int32_t* order, int64_t lanes_per_ray, void* work, int64_t work_bytes,
                                       void* stream) {
    using namespace vgr;
    VGR_REQUIRE(lanes_per_ray == 0 || lanes_per_ray == 1 || lanes_per_ray == kGroup,
                "march_forward: lanes_per_ray must be 0 (by batch size), 1 or 16 (got %lld)",
                static_cast<long long>(lanes_per_ray));
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
    const int64_t need = vgr_march_work_size(n_sites, sh_deg);
    VGR_REQUIRE(work && work_bytes >= need, "march_forward: work must hold %lld bytes", static_cast<long long>(need));
    VGR_REQUIRE(reinterpret_cast<uintptr_t>(work) % 256 == 0, "march_forward: work must be 256-byte aligned");
    float4* rec = static_cast<float4*>(work);
    launch_pack(points, raw, dA, cA, sh, n_sites, sh_deg, rec, as_stream(stream));
    const MarchField F{rec, offsets, adj, int(sh_deg), int(n_sites)};
    const MarchParams M{float(dt), int(n_bg), float(t_thresh), float(w_thresh)};
    const MarchRays R{o, d, start, near_t, mid_t, far_t, n_rays, order};
    const MarchOut O{rgb, T, depth, stats, trace, trace_cap};
    if (march_lanes(lanes_per_ray, n_rays) == kGroup) {
        const dim3 grid(grid_for(n_rays * kGroup, kBlock));
        if (trace != nullptr)
            hipLaunchKernelGGL(march_group_kernel<true>, grid, dim3(kBlock), 0, as_stream(stream), F, M, R, O);
        else
            hipLaunchKernelGGL(march_group_kernel<false>, grid, dim3(kBlock), 0, as_stream(stream), F, M, R, O);
        return launch_status("march_group_kernel");
    }
    if (trace != nullptr)
        hipLaunchKernelGGL(march_forward_kernel<true>, dim3(grid_for(n_rays, kBlock)), dim3(kBlock), 0,
                           as_stream(stream), F, M, R, O);
    else
        hipLaunchKernelGGL(march_forward_kernel<false>, dim3(grid_for(n_rays, kBlock)), dim3(kBlock), 0,
                           as_stream(stream), F, M, R, O);
    return launch_status("march_forward_kernel");
}

extern "C" int vgr_march_forward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                                 int64_t n_adj, const float* raw, const float* dA, const float* cA, const float* sh,
                                 int64_t sh_deg, const float* o, const float* d, const int32_t* start,
                                 const float* near_t, const float* mid_t, const float* far_t, int64_t n_rays,
                                 double dt, int64_t n_bg, double t_thresh, double w_thresh, float* rgb, float* T,
                                 float* depth, int32_t* stats, int32_t* trace, int64_t trace_cap, void* work,
                                 int64_t work_bytes, void* stream) {
    return vgr_march_forward_lanes(points, n_sites, offsets, adj, n_adj, raw, dA, cA, sh, sh_deg, o, d, start, near_t,
                                   mid_t, far_t, n_rays, dt, n_bg, t_thresh, w_thresh, rgb, T, depth, stats, trace,
                                   trace_cap, nullptr, 0, work, work_bytes, stream);
}

extern "C" int vgr_march_backward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                                  int64_t n_adj, const float* raw, const float* dA, const float* cA, const float* sh,
                                  int64_t sh_deg, const float* o, const float* d, const int32_t* start,
                                  const float* near_t, const float* mid_t, const float* far_t, int64_t n_rays,
                                  double dt, int64_t n_bg, double t_thresh, double w_thresh, const float* rgb,
                                  const float* T, const float* g_rgb, const float* g_T, float* g_raw, float* g_dA,
                                  float* g_cA, float* g_sh, int64_t lanes_per_ray, int64_t blocks_ready, void* work,
                                  int64_t work_bytes, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(lanes_per_ray == 0 || lanes_per_ray == 1 || lanes_per_ray == kGroup,
                "march_backward: lanes_per_ray must be 0 (by batch size), 1 or 16 (got %lld)",
                static_cast<long long>(lanes_per_ray));
    VGR_REQUIRE(n_rays >= 0, "march_backward: n_rays must be >= 0 (got %lld)", static_cast<long long>(n_rays));
    VGR_REQUIRE(sh_deg >= 0 && sh_deg <= 3, "sh_deg must be in [0, 3] (got %lld)", static_cast<long long>(sh_deg));
    VGR_REQUIRE(n_bg >= 0 && n_bg <= INT_MAX, "march_backward: n_bg must be >= 0");
    VGR_REQUIRE(dt > 0.0, "march_backward: dt must be > 0");
    VGR_REQUIRE(n_sites > 0 && n_sites <= INT_MAX, "march_backward: n_sites must be in [1, 2^31)");
    VGR_REQUIRE(n_adj >= 0 && n_adj <= INT_MAX, "march_backward: n_adj must be in [0, 2^31)");
    VGR_REQUIRE(g_raw && g_dA && g_cA && g_sh, "march_backward: null gradient pointer");
    const hipStream_t s = as_stream(stream);
    // the gradients are overwritten (zeroed by a kernel, not a memset, so a captured stream records no memset node)
    if (n_rays == 0) {
        float* const outs[4] = {g_raw, g_dA, g_cA, g_sh};
        const int64_t sizes[4] = {n_sites, 6 * n_sites, 6 * n_sites, 48 * n_sites};
        for (int u = 0; u < 4; ++u)
            hipLaunchKernelGGL(zero_kernel, dim3(kZeroBlocks), dim3(256), 0, s, outs[u], sizes[u]);
        return launch_status("march_backward zero");
    }
    VGR_REQUIRE(points && offsets && (adj || n_adj == 0) && raw && dA && cA && sh,
                "march_backward: null field pointer");
    VGR_REQUIRE(o && d && start && near_t && mid_t && far_t, "march_backward: null ray pointer");
    VGR_REQUIRE(rgb && T && g_rgb && g_T, "march_backward: null forward output or upstream gradient pointer");
    const int64_t need = vgr_march_backward_work_size(n_sites, sh_deg);
    VGR_REQUIRE(work && work_bytes >= need, "march_backward: work must hold %lld bytes", static_cast<long long>(need));
    VGR_REQUIRE(reinterpret_cast<uintptr_t>(work) % 256 == 0, "march_backward: work must be 256-byte aligned");
    float4* rec = static_cast<float4*>(work);
    if (!blocks_ready) launch_pack(points, raw, dA, cA, sh, n_sites, sh_deg, rec, s);
    const MarchField F{rec, offsets, adj, int(sh_deg), int(n_sites)};
    const MarchParams M{float(dt), int(n_bg), float(t_thresh), float(w_thresh)};
    const MarchRays R{o, d, start, near_t, mid_t, far_t, n_rays};
    const MarchGradIn GI{rgb, T, g_rgb, g_T};
    float* block = reinterpret_cast<float*>(static_cast<char*>(work) + vgr_march_work_size(n_sites, sh_deg));
    hipLaunchKernelGGL(zero_kernel, dim3(kZeroBlocks), dim3(256), 0, s, block, kGradBlock * n_sites);
    const MarchGradOut G{block};
    // wave-shared atomics once the launch holds at least one wave per CU (16384 rays); per-lane atomics below, where
    // the launch is bound by the latency of its few waves (config 5: 4096 rays 85 against 158 ms, 65536 rays 456
    // against 193 ms)
    if (march_lanes(lanes_per_ray, n_rays) == kGroup)
        hipLaunchKernelGGL(march_group_backward_kernel, dim3(grid_for(n_rays * kGroup, kBlock)), dim3(kBlock), 0, s,
                           F, M, R, GI, G);
    else if (n_rays >= kCoopRays)
        hipLaunchKernelGGL(march_backward_kernel<true>, dim3(grid_for(n_rays, kBlock)), dim3(kBlock), 0, s, F, M, R,
                           GI, G);
    else
        hipLaunchKernelGGL(march_backward_kernel<false>, dim3(grid_for(n_rays, kBlock)), dim3(kBlock), 0, s, F, M, R,
                           GI, G);
    hipLaunchKernelGGL(grad_unpack_kernel, dim3(grid_for(kGradBlock * n_sites, 256)), dim3(256), 0, s, block, n_sites,
                       g_raw, g_dA, g_cA, g_sh);
    return launch_status("march_backward_kernel");
}

extern "C" int64_t vgr_foam_work_size(int64_t n_sites, int64_t sh_deg) {
    return vgr_march_backward_work_size(n_sites, sh_deg);
}

namespace vgr {
namespace {
int train_check(int64_t n_sites, int64_t n_adj, int64_t sh_deg, int64_t n_rays, int64_t record_cap, const void* work,
                int64_t work_bytes, const char* who) {
    VGR_REQUIRE(n_rays >= 0, "%s: n_rays must be >= 0 (got %lld)", who, static_cast<long long>(n_rays));
    VGR_REQUIRE(sh_deg >= 0 && sh_deg <= 3, "sh_deg must be in [0, 3] (got %lld)", static_cast<long long>(sh_deg));
    VGR_REQUIRE(record_cap >= 0 && record_cap <= INT_MAX, "%s: record_cap must be in [0, 2^31)", who);
    VGR_REQUIRE(n_sites > 0 && n_sites <= INT_MAX, "%s: n_sites must be in [1, 2^31)", who);
    VGR_REQUIRE(n_adj >= 0 && n_adj <= INT_MAX, "%s: n_adj must be in [0, 2^31)", who);
    const int64_t need = vgr_foam_work_size(n_sites, sh_deg);
    VGR_REQUIRE(work && work_bytes >= need, "%s: work must hold %lld bytes", who, static_cast<long long>(need));
    VGR_REQUIRE(reinterpret_cast<uintptr_t>(work) % 256 == 0, "%s: work must be 256-byte aligned", who);
    return VGR_OK;
}
}  // namespace
}  // namespace vgr

extern "C" int vgr_foam_forward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                                int64_t n_adj, const float* raw, const float* dA, const float* cA, const float* sh,
                                int64_t sh_deg, const float* o, const float* d, const int32_t* start,
                                const float* near_t, const float* far_t, int64_t n_rays, double t_thresh,
                                double w_thresh, float* rgb, float* T, float* depth, int32_t* stats, float* rec,
                                int64_t record_cap, void* work, int64_t work_bytes, void* stream) {
    using namespace vgr;
    if (n_rays == 0) {
        VGR_REQUIRE(record_cap >= 0, "foam_forward: record_cap must be >= 0");
        return VGR_OK;
    }
    const int st = train_check(n_sites, n_adj, sh_deg, n_rays, record_cap, work, work_bytes, "foam_forward");
    if (st != VGR_OK) return st;
    VGR_REQUIRE(points && offsets && (adj || n_adj == 0) && raw && dA && cA && sh, "foam_forward: null field pointer");
    VGR_REQUIRE(o && d && start && near_t && far_t, "foam_forward: null ray pointer");
    VGR_REQUIRE(rgb && T && depth && stats, "foam_forward: null output pointer");
    VGR_REQUIRE(record_cap == 0 || rec, "foam_forward: record_cap > 0 needs rec");
    const hipStream_t s = as_stream(stream);
    float4* recb = static_cast<float4*>(work);
    launch_pack(points, raw, dA, cA, sh, n_sites, sh_deg, recb, s);
    const MarchField F{recb, offsets, adj, int(sh_deg), int(n_sites)};
    const MarchParams M{1.f, 0, float(t_thresh), float(w_thresh)};
    const TrainRays R{o, d, start, near_t, far_t, n_rays};
    const MarchOut O{rgb, T, depth, stats, nullptr, 0};
    hipLaunchKernelGGL(train_forward_kernel, dim3(grid_for(n_rays * kGroup, kBlock)), dim3(kBlock), 0, s, F, M, R, O,
                       record_cap > 0 ? rec : nullptr, int(record_cap));
    return launch_status("train_forward_kernel");
}

extern "C" int vgr_foam_backward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                                 int64_t n_adj, const float* raw, const float* dA, const float* cA, const float* sh,
                                 int64_t sh_deg, const float* o, const float* d, const int32_t* start,
                                 const float* near_t, const float* far_t, int64_t n_rays, double t_thresh,
                                 double w_thresh, const float* rgb, const float* T, const float* g_rgb,
                                 const float* g_T, const float* rec, int64_t record_cap, const int32_t* stats,
                                 float* g_raw, float* g_dA, float* g_cA, float* g_sh, int64_t blocks_ready,
                                 void* work, int64_t work_bytes, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(n_sites > 0 && n_sites <= INT_MAX, "foam_backward: n_sites must be in [1, 2^31)");
    VGR_REQUIRE(g_raw && g_dA && g_cA && g_sh, "foam_backward: null gradient pointer");
    const hipStream_t s = as_stream(stream);
    if (n_rays == 0) {
        float* const outs[4] = {g_raw, g_dA, g_cA, g_sh};
        const int64_t sizes[4] = {n_sites, 6 * n_sites, 6 * n_sites, 48 * n_sites};
        for (int u = 0; u < 4; ++u)
            hipLaunchKernelGGL(zero_kernel, dim3(kZeroBlocks), dim3(256), 0, s, outs[u], sizes[u]);
        return launch_status("foam_backward zero");
    }
    const int st = train_check(n_sites, n_adj, sh_deg, n_rays, record_cap, work, work_bytes, "foam_backward");
    if (st != VGR_OK) return st;
    VGR_REQUIRE(points && offsets && (adj || n_adj == 0) && raw && dA && cA && sh, "foam_backward: null field pointer");
    VGR_REQUIRE(o && d && start && near_t && far_t, "foam_backward: null ray pointer");
    VGR_REQUIRE(rgb && T && g_rgb && g_T, "foam_backward: null forward output or upstream gradient pointer");
    VGR_REQUIRE(record_cap == 0 || (rec && stats), "foam_backward: records need rec and the forward's stats");
    float4* recb = static_cast<float4*>(work);
    if (!blocks_ready) launch_pack(points, raw, dA, cA, sh, n_sites, sh_deg, recb, s);
    float* block = reinterpret_cast<float*>(static_cast<char*>(work) + vgr_march_work_size(n_sites, sh_deg));
    hipLaunchKernelGGL(zero_kernel, dim3(kZeroBlocks), dim3(256), 0, s, block, kGradBlock * n_sites);
    const MarchField F{recb, offsets, adj, int(sh_deg), int(n_sites)};
    const MarchParams M{1.f, 0, float(t_thresh), float(w_thresh)};
    const TrainRays R{o, d, start, near_t, far_t, n_rays};
    const MarchGradIn GI{rgb, T, g_rgb, g_T};
    const MarchGradOut G{block};
    hipLaunchKernelGGL(train_backward_kernel, dim3(grid_for(n_rays * kGroup, kBlock)), dim3(kBlock), 0, s, F, M, R,
                       GI, G, record_cap > 0 ? rec : nullptr, int(record_cap), stats);
    hipLaunchKernelGGL(grad_unpack_kernel, dim3(grid_for(kGradBlock * n_sites, 256)), dim3(256), 0, s, block, n_sites,
                       g_raw, g_dA, g_cA, g_sh);
    return launch_status("train_backward_kernel");
}
