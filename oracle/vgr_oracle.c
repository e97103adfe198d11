/*
 * CPU oracle of the voronoi-gauss forward/inference path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file is the parity checker and the reported CPU baseline. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load it; the product path (libvgr.so) never links, loads or calls it.
 *
 * It restates, in plain C with a declared fp32 arithmetic, the semantics of the reference kernels:
 *   foam_infer    csrc/foam_infer.cu:50-361   (walk_to :176-194, eval_cell :199-257, color_lazy :260-284,
 *                                               kernel :286-361, cache :151-168, site_color :121-149)
 *   march_forward csrc/march.cu:134-262        (load_ray :134-141, sample_at :143-153, walk_to :157-180,
 *                                               density_at :182-192, color_at :195-219, kernel :221-262)
 *   march_backward csrc/march.cu:264-345, 402-428
 *   training renderer (foam.cu) forward and backward   csrc/foam.cu:160-469
 *   walk          csrc/vgf.cu:51-79
 *   density       csrc/vgf.cu:98-119,152-177
 *   color         csrc/vgf.cu:202-282
 *   conic         csrc/vgf.cu:340-380
 *   density, color and conic backward   csrc/vgf.cu:121-148,179-198,284-333,382-424
 * Arithmetic contract shared with the HIP kernels: fp32, every expression evaluated left to right as
 * written, no contraction into FMA (-ffp-contract=off), IEEE division and sqrt, fminf/fmaxf. Transcendentals
 * (expf) are libm's; the kernels call the device exp, so values agree to a few ulps, not bitwise.
 * The visited-cell sequences depend only on comparisons of non-contracted products/sums and one division,
 * which both sides evaluate identically, so they agree bit for bit.
 *
 * Pinning (what checks this file, tests/test_oracle.py): float64 dense references restated from the
 * reference tests (test_foam.py:18-37,76-104; test_march.py:14-22,59-79; test_grad.py:21-48,92-104),
 * brute-force nearest sites, the segment-in-cell invariant, closed forms (SH constants at d=(0,0,1), conic
 * A*Sigma = I), lazy == fused colours, cache on == cache off, Morton-renumbering invariance.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <limits.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define K_INF 3.402823466e38f
#define K_WALK_CAP 4096
#define K_MAX_CELLS 8192
#define K_CACHE 8

enum { LAZY = 0, BAKED = 1, FUSED = 2 };

/* ------------------------------------------------------------------------------------------ helpers */

/* IEEE binary16 -> binary32, exact (every half is a float). */
static float half_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else { /* subnormal half: m * 2^-24 */
            float f = (float)m * 5.9604644775390625e-08f;
            memcpy(&bits, &f, 4);
            bits |= s;
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 112) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

static inline float bits_float(int32_t i) { float f; memcpy(&f, &i, 4); return f; }
static inline int32_t float_bits(float f) { int32_t i; memcpy(&i, &f, 4); return i; }

/* (r2, lam) stored as half2 in the 4th float of an edge record: low half r2, high half lam (render.py:197). */
static inline void cutoffs(float w, float* r2, float* lam) {
    uint32_t u;
    memcpy(&u, &w, 4);
    *r2 = half_to_float((uint16_t)(u & 0xffffu));
    *lam = half_to_float((uint16_t)(u >> 16));
}

/* v^T A v with A = (xx, xy, xz, yy, yz, zz); foam_infer.cu:74-77, march.cu:80-84. */
static inline float maha(float xx, float xy, float xz, float yy, float yz, float zz, float vx, float vy, float vz) {
    return xx * vx * vx + yy * vy * vy + zz * vz * vz + 2.f * (xy * vx * vy + xz * vx * vz + yz * vy * vz);
}

/* Real SH basis, 3DGS constants and signs; foam_infer.cu:95-118 = march.cu:97-120 = vgf.cu:205-228. */
static void sh_basis(float x, float y, float z, int deg, float b[16]) {
    b[0] = 0.28209479177387814f;
    for (int i = 1; i < 16; ++i) b[i] = 0.f;
    if (deg < 1) return;
    b[1] = -0.4886025119029199f * y;
    b[2] = 0.4886025119029199f * z;
    b[3] = -0.4886025119029199f * x;
    if (deg < 2) return;
    const float xx = x * x, yy = y * y, zz = z * z;
    b[4] = 1.0925484305920792f * x * y;
    b[5] = -1.0925484305920792f * y * z;
    b[6] = 0.31539156525252005f * (2.f * zz - xx - yy);
    b[7] = -1.0925484305920792f * x * z;
    b[8] = 0.5462742152960396f * (xx - yy);
    if (deg < 3) return;
    b[9] = -0.5900435899266435f * y * (3.f * xx - yy);
    b[10] = 2.890611442640554f * x * y * z;
    b[11] = -0.4570457994644658f * y * (4.f * zz - xx - yy);
    b[12] = 0.3731763325901154f * z * (2.f * zz - 3.f * xx - 3.f * yy);
    b[13] = -0.4570457994644658f * x * (4.f * zz - xx - yy);
    b[14] = 1.445305721320277f * z * (xx - yy);
    b[15] = -0.5900435899266435f * x * (xx - 3.f * yy);
}

void oracle_sh_basis(float x, float y, float z, int deg, float* b) { sh_basis(x, y, z, deg, b); }

/* ======================================================================================= foam_infer */

typedef struct {
    const float* points;   /* (N, 4) */
    const int32_t* offsets; /* (N + 1), self-first neighbourhoods */
    const int32_t* nbr;    /* (E) */
    const float* edge;     /* (E, 4): p_j, half2(r2_j, lam_j) */
    const float* attr;     /* (N, 20) */
    const void* sh;        /* (N, 16, 3) f32 or f16 */
    const int32_t* orig;   /* (N) or NULL */
    int sh_half;
} Net;

typedef struct {
    float t_thresh, w_thresh, color_cut;
    int sh_deg, color_mode, stage, use_cache;
} Opt;

typedef struct { float m, a, r, g, b; } Blend;

typedef struct { float rgb[3]; int key; } Slot;

/* k precedes j in the tie-breaking order (smaller original index); foam_infer.cu:61-63. */
static inline int before(const Net* N, int k, int j) {
    return N->orig != NULL ? N->orig[k] < N->orig[j] : k < j;
}

static inline void blend_init(Blend* B) { B->m = K_INF; B->a = B->r = B->g = B->b = 0.f; }

/* Online normalised blend; foam_infer.cu:81-88. */
static inline void blend_add(Blend* B, float m, float r, float g, float b) {
    if (m < B->m) {
        const float s = expf(-0.5f * (B->m - m));
        B->a *= s; B->r *= s; B->g *= s; B->b *= s; B->m = m;
    }
    const float w = expf(-0.5f * (m - B->m));
    B->a += w; B->r += w * r; B->g += w * g; B->b += w * b;
}

/* max(SH_k(d) + 1/2, 0) over all 48 coefficients in storage order; foam_infer.cu:121-149. */
static void site_color(const Net* N, int k, const float b[16], float c[3]) {
    c[0] = c[1] = c[2] = 0.5f;
    if (N->sh_half) {
        const uint16_t* s = (const uint16_t*)N->sh + 48 * (int64_t)k;
        for (int i = 0; i < 48; ++i) c[i % 3] += b[i / 3] * half_to_float(s[i]);
    } else {
        const float* s = (const float*)N->sh + 48 * (int64_t)k;
        for (int i = 0; i < 48; ++i) c[i % 3] += b[i / 3] * s[i];
    }
    c[0] = fmaxf(c[0], 0.f); c[1] = fmaxf(c[1], 0.f); c[2] = fmaxf(c[2], 0.f);
}

/* Per-ray direct-mapped colour cache, slot k mod 8; foam_infer.cu:151-168. With use_cache = 0 every lookup
 * misses, which must give identical colours (only the SH-evaluation counter changes). */
static void cached_color(const Net* N, const Opt* M, Slot* cache, int k, const float b[16], float c[3], int* n_sh) {
    Slot* e = &cache[k & (K_CACHE - 1)];
    if (M->use_cache && e->key == k) {
        c[0] = e->rgb[0]; c[1] = e->rgb[1]; c[2] = e->rgb[2];
        return;
    }
    site_color(N, k, b, c);
    e->rgb[0] = c[0]; e->rgb[1] = c[1]; e->rgb[2] = c[2]; e->key = k;
    ++*n_sh;
}

/* Greedy walk to the lexicographic argmin of (|x - p|^2, tie order) over {c} U adj(c); foam_infer.cu:176-194. */
static int foam_walk_to(const Net* N, int c, float x0, float x1, float x2, int* steps) {
    for (int it = 0; it < K_WALK_CAP; ++it) {
        const float* pc = N->points + 4 * (int64_t)c;
        float bd = (x0 - pc[0]) * (x0 - pc[0]) + (x1 - pc[1]) * (x1 - pc[1]) + (x2 - pc[2]) * (x2 - pc[2]);
        int bk = c;
        const int e0 = N->offsets[c], e1 = N->offsets[c + 1];
        for (int e = e0 + 1; e < e1; ++e) {
            const float* ed = N->edge + 4 * (int64_t)e;
            const int k = N->nbr[e];
            const float v0 = x0 - ed[0], v1 = x1 - ed[1], v2 = x2 - ed[2];
            const float dk = v0 * v0 + v1 * v1 + v2 * v2;
            if (dk < bd || (dk == bd && before(N, k, bk))) { bd = dk; bk = k; }
        }
        if (bk == c) break;
        c = bk;
        ++*steps;
    }
    return c;
}

/* One pass over the self-first neighbourhood of cell c for the sample at o + t d; foam_infer.cu:199-257. */
static void eval_cell(const Net* N, const Opt* M, int c, float t, const float o[3], const float d[3],
                      const float b[16], Slot* cache, int want_exit, float* sigma, float* mmin, Blend* B,
                      float* t_exit, int* next, int* n_dens, int* n_sh) {
    const int blend = M->color_mode != LAZY;
    const float* pc = N->points + 4 * (int64_t)c;
    const float x0 = o[0] + t * d[0], x1 = o[1] + t * d[1], x2 = o[2] + t * d[2];
    const int e0 = N->offsets[c], e1 = N->offsets[c + 1];
    *sigma = 0.f; *mmin = K_INF;
    blend_init(B);
    *t_exit = K_INF; *next = INT_MAX;
    for (int e = e0; e < e1; ++e) {
        const float* ed = N->edge + 4 * (int64_t)e;
        const int k = N->nbr[e];
        if (want_exit && e > e0) {
            const float n0 = ed[0] - pc[0], n1 = ed[1] - pc[1], n2 = ed[2] - pc[2];
            const float dn = n0 * d[0] + n1 * d[1] + n2 * d[2];
            if (dn > 0.f) {
                const float m0 = 0.5f * (ed[0] + pc[0]) - o[0], m1 = 0.5f * (ed[1] + pc[1]) - o[1],
                            m2 = 0.5f * (ed[2] + pc[2]) - o[2];
                const float tt = (m0 * n0 + m1 * n1 + m2 * n2) / dn;
                if (tt < *t_exit || (tt == *t_exit && (*next == INT_MAX || before(N, k, *next)))) {
                    *t_exit = tt; *next = k;
                }
            }
        }
        if (M->stage >= 1) {
            const float v0 = x0 - ed[0], v1 = x1 - ed[1], v2 = x2 - ed[2];
            const float r2 = v0 * v0 + v1 * v1 + v2 * v2;
            float cut_r2, cut_lam;
            cutoffs(ed[3], &cut_r2, &cut_lam);
            const float* a = N->attr + 20 * (int64_t)k;
            if (r2 <= cut_r2) {
                *sigma += expf(a[6] - 0.5f * maha(a[0], a[1], a[2], a[3], a[4], a[5], v0, v1, v2));
                ++*n_dens;
            }
            if (M->stage >= 2) {
                const float lb = r2 * cut_lam;
                if (blend ? lb <= B->m + M->color_cut : lb < *mmin) {
                    const float m = maha(a[8], a[9], a[10], a[11], a[12], a[13], v0, v1, v2);
                    if (blend) {
                        if (m <= B->m + M->color_cut) {
                            float c3[3];
                            if (M->color_mode == BAKED) {
                                c3[0] = a[16]; c3[1] = a[17]; c3[2] = a[18];
                            } else {
                                cached_color(N, M, cache, k, b, c3, n_sh);
                            }
                            blend_add(B, m, c3[0], c3[1], c3[2]);
                        }
                    } else {
                        *mmin = fminf(*mmin, m);
                    }
                }
            }
        }
    }
}

/* Second (colour) pass of the lazy mode; foam_infer.cu:260-284. */
static void color_lazy(const Net* N, const Opt* M, int c, float t, float mmin, const float o[3], const float d[3],
                       const float b[16], Slot* cache, float C[3], int* n_sh) {
    const float x0 = o[0] + t * d[0], x1 = o[1] + t * d[1], x2 = o[2] + t * d[2];
    const int e0 = N->offsets[c], e1 = N->offsets[c + 1];
    const float cut = mmin + M->color_cut;
    float A = 0.f, r = 0.f, g = 0.f, bl = 0.f;
    for (int e = e0; e < e1; ++e) {
        const float* ed = N->edge + 4 * (int64_t)e;
        const float v0 = x0 - ed[0], v1 = x1 - ed[1], v2 = x2 - ed[2];
        float cut_r2, cut_lam;
        cutoffs(ed[3], &cut_r2, &cut_lam);
        if ((v0 * v0 + v1 * v1 + v2 * v2) * cut_lam > cut) continue;
        const int k = N->nbr[e];
        const float* a = N->attr + 20 * (int64_t)k;
        const float m = maha(a[8], a[9], a[10], a[11], a[12], a[13], v0, v1, v2);
        if (m > cut) continue;
        const float w = expf(-0.5f * (m - mmin));
        float c3[3];
        cached_color(N, M, cache, k, b, c3, n_sh);
        A += w; r += w * c3[0]; g += w * c3[1]; bl += w * c3[2];
    }
    const float inv = 1.f / A;
    C[0] = r * inv; C[1] = g * inv; C[2] = bl * inv;
}

/* One ray of foam_infer_kernel (foam_infer.cu:286-361). trace (optional) receives the cell of every sample,
 * in original numbering, up to trace_cap entries; the sample count is stats[0]. */
static void foam_ray(const Net* N, const Opt* M, const float o[3], const float d[3], int start, float t_near,
                     float t_far, int max_samples, float rgb[3], float* T_out, float* depth, int32_t stats[5],
                     int32_t* trace, int trace_cap) {
    const int blend = M->stage >= 2 && M->color_mode != LAZY;
    Slot cache[K_CACHE];
    for (int i = 0; i < K_CACHE; ++i) { cache[i].rgb[0] = cache[i].rgb[1] = cache[i].rgb[2] = 0.f; cache[i].key = -1; }
    float b[16];
    for (int i = 0; i < 16; ++i) b[i] = 0.f;
    if (M->stage >= 2 && M->color_mode != BAKED) sh_basis(d[0], d[1], d[2], M->sh_deg, b);

    int walk_steps = 0, n_dens = 0, n_sh = 0;
    int c = foam_walk_to(N, start, o[0] + t_near * d[0], o[1] + t_near * d[1], o[2] + t_near * d[2], &walk_steps);
    float sP, mP, t_exit;
    int next;
    Blend BP, BQ;
    eval_cell(N, M, c, t_near, o, d, b, cache, 1, &sP, &mP, &BP, &t_exit, &next, &n_dens, &n_sh);
    if (trace != NULL && trace_cap > 0) trace[0] = N->orig != NULL ? N->orig[c] : c;
    float tP = t_near, CP[3] = {0.f, 0.f, 0.f};
    int hasP = 0, cP = c;
    if (blend) {
        const float inv = 1.f / BP.a;
        CP[0] = BP.r * inv; CP[1] = BP.g * inv; CP[2] = BP.b * inv; hasP = 1;
    }
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f}, dep = 0.f;
    int n_samples = 1, n_color = 0;
    for (int it = 0; it < K_MAX_CELLS; ++it) {
        const int last = next == INT_MAX || t_exit >= t_far || n_samples + 1 >= max_samples;
        const float tQ = last ? t_far : fmaxf(t_exit, tP);
        const int cQ = last ? c : next;
        float sQ, mQ;
        eval_cell(N, M, cQ, tQ, o, d, b, cache, !last, &sQ, &mQ, &BQ, &t_exit, &next, &n_dens, &n_sh);
        if (trace != NULL && n_samples < trace_cap) trace[n_samples] = N->orig != NULL ? N->orig[cQ] : cQ;
        ++n_samples;
        const float delta = tQ - tP;
        const float alpha = 1.f - expf(-0.5f * (sP + sQ) * delta);
        const float w = T * alpha;
        float CQ[3] = {0.f, 0.f, 0.f};
        int hasQ = 0;
        if (blend) {
            const float inv = 1.f / BQ.a;
            CQ[0] = BQ.r * inv; CQ[1] = BQ.g * inv; CQ[2] = BQ.b * inv; hasQ = 1;
        }
        if (M->stage >= 2 && w > M->w_thresh) {
            if (!blend) {
                if (!hasP) color_lazy(N, M, cP, tP, mP, o, d, b, cache, CP, &n_sh);
                color_lazy(N, M, cQ, tQ, mQ, o, d, b, cache, CQ, &n_sh);
                hasQ = 1;
            }
            for (int a = 0; a < 3; ++a) acc[a] += w * 0.5f * (CP[a] + CQ[a]);
            dep += w * 0.5f * (tP + tQ);
            ++n_color;
        }
        T *= 1.f - alpha;
        tP = tQ; sP = sQ; mP = mQ; hasP = hasQ; cP = cQ; c = cQ;
        for (int a = 0; a < 3; ++a) CP[a] = CQ[a];
        if (last || T < M->t_thresh) break;
    }
    for (int a = 0; a < 3; ++a) rgb[a] = acc[a];
    *T_out = T;
    *depth = dep;
    stats[0] = n_samples; stats[1] = n_color; stats[2] = walk_steps; stats[3] = n_dens; stats[4] = n_sh;
}

/* Renders the rays listed in `rays` (or all B rays when rays == NULL, n_sel = B) on n_threads OpenMP threads.
 * Outputs are indexed by the position in the selection. Returns the wall time in seconds of the parallel loop. */
double oracle_foam_infer(const float* points, const int32_t* offsets, const int32_t* nbr, const float* edge,
                         const float* attr, const void* sh, int sh_half, int sh_deg, const float* o, const float* d,
                         const int32_t* start, const float* near_t, const float* far_t, const int64_t* rays,
                         int64_t n_sel, float t_thresh, float w_thresh, float color_cut, int color_mode, int stage,
                         const int32_t* cap, const int32_t* orig, int use_cache, float* rgb, float* T, float* depth,
                         int32_t* stats, int32_t* trace, int trace_cap, int n_threads) {
    const Net N = {points, offsets, nbr, edge, attr, sh, orig, sh_half};
    const Opt M = {t_thresh, w_thresh, color_cut, sh_deg, color_mode, stage, use_cache};
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
    const double t0 = omp_get_wtime();
#pragma omp parallel for schedule(dynamic, 256)
#endif
    for (int64_t i = 0; i < n_sel; ++i) {
        const int64_t r = rays != NULL ? rays[i] : i;
        const int ms = cap != NULL ? cap[r] : INT_MAX;
        foam_ray(&N, &M, o + 3 * r, d + 3 * r, start[r], near_t[r], far_t[r], ms, rgb + 3 * i, T + i, depth + i,
                 stats + 5 * i, trace != NULL ? trace + (int64_t)trace_cap * i : NULL, trace_cap);
    }
#ifdef _OPENMP
    return omp_get_wtime() - t0;
#else
    return 0.0;
#endif
}

/* ==================================================================================== march_forward */

typedef struct {
    const float* points;   /* (N, 3) */
    const int32_t* offsets; /* (N + 1) */
    const int32_t* adj;    /* (M) */
    const float* raw, *dA, *cA, *sh;
    int sh_deg;
} Field;

static inline int neighbor(const Field* F, int i, int e0, int e) { return e == 0 ? i : F->adj[e0 + e - 1]; }

/* Sample k of a ray: midpoints of dt steps to mid, then n_bg steps uniform in disparity; march.cu:143-153. */
static void sample_at(float near, float mid, float far, int n_in, float dt, int n_bg, int k, float* t, float* delta) {
    if (k < n_in) {
        const float t0 = near + (float)k * dt, t1 = fminf(t0 + dt, mid);
        *t = 0.5f * (t0 + t1);
        *delta = t1 - t0;
    } else {
        const float i0 = 1.f / mid, i1 = 1.f / far;
        const float u0 = (float)(k - n_in) / (float)n_bg, u1 = (float)(k - n_in + 1) / (float)n_bg;
        *t = 1.f / (i0 + 0.5f * (u0 + u1) * (i1 - i0));
        *delta = 1.f / (i0 + u1 * (i1 - i0)) - 1.f / (i0 + u0 * (i1 - i0));
    }
}

void oracle_sample_at(float near, float mid, float far, int n_in, float dt, int n_bg, int k, float* t, float* delta) {
    sample_at(near, mid, far, n_in, dt, n_bg, k, t, delta);
}

/* Lexicographic argmin of (|x - p|^2, index) over {cur} U adj(cur), repeated; march.cu:157-180. */
static int march_walk_to(const Field* F, int cur, const float x[3], int* steps) {
    for (int it = 0; it < K_WALK_CAP; ++it) {
        const int e0 = F->offsets[cur], n = F->offsets[cur + 1] - e0 + 1;
        float bd = K_INF;
        int bk = INT_MAX;
        for (int e = 0; e < n; ++e) {
            const int k = neighbor(F, cur, e0, e);
            const float* p = F->points + 3 * (int64_t)k;
            const float v0 = x[0] - p[0], v1 = x[1] - p[1], v2 = x[2] - p[2];
            const float dk = v0 * v0 + v1 * v1 + v2 * v2;
            if (dk < bd || (dk == bd && k < bk)) { bd = dk; bk = k; }
        }
        if (bk == cur) break;
        cur = bk;
        ++*steps;
    }
    return cur;
}

static inline float conic_maha(const float* A, int k, const float v[3]) {
    const float* a = A + 6 * (int64_t)k;
    return a[0] * v[0] * v[0] + a[3] * v[1] * v[1] + a[5] * v[2] * v[2] +
           2.f * (a[1] * v[0] * v[1] + a[2] * v[0] * v[2] + a[4] * v[1] * v[2]);
}

static void sh_eval(const float* sh, int k, const float b[16], int nb, float c[3]) {
    const float* p = sh + 48 * (int64_t)k;
    c[0] = c[1] = c[2] = 0.5f;
    for (int j = 0; j < 16 && j < nb; ++j) {
        c[0] += b[j] * p[3 * j];
        c[1] += b[j] * p[3 * j + 1];
        c[2] += b[j] * p[3 * j + 2];
    }
}

/* Density at x over the neighbourhood of i (sequential sum); march.cu:182-192. */
static float march_density(const Field* F, int i, const float x[3]) {
    const int e0 = F->offsets[i], n = F->offsets[i + 1] - e0 + 1;
    float s = 0.f;
    for (int e = 0; e < n; ++e) {
        const int k = neighbor(F, i, e0, e);
        const float* p = F->points + 3 * (int64_t)k;
        const float v[3] = {x[0] - p[0], x[1] - p[1], x[2] - p[2]};
        s += expf(fminf(F->raw[k], 30.f) - 0.5f * conic_maha(F->dA, k, v));
    }
    return s;
}

/* Two-pass normalised colour blend; march.cu:195-219. */
static void march_color(const Field* F, int i, const float x[3], const float b[16], float C[3]) {
    const int e0 = F->offsets[i], n = F->offsets[i + 1] - e0 + 1;
    const int nb = (F->sh_deg + 1) * (F->sh_deg + 1);
    float mmin = K_INF;
    for (int e = 0; e < n; ++e) {
        const int k = neighbor(F, i, e0, e);
        const float* p = F->points + 3 * (int64_t)k;
        const float v[3] = {x[0] - p[0], x[1] - p[1], x[2] - p[2]};
        mmin = fminf(mmin, conic_maha(F->cA, k, v));
    }
    float A = 0.f, cr = 0.f, cg = 0.f, cb = 0.f;
    for (int e = 0; e < n; ++e) {
        const int k = neighbor(F, i, e0, e);
        const float* p = F->points + 3 * (int64_t)k;
        const float v[3] = {x[0] - p[0], x[1] - p[1], x[2] - p[2]};
        const float a = expf(-0.5f * (conic_maha(F->cA, k, v) - mmin));
        float c[3];
        sh_eval(F->sh, k, b, nb, c);
        A += a; cr += a * fmaxf(c[0], 0.f); cg += a * fmaxf(c[1], 0.f); cb += a * fmaxf(c[2], 0.f);
    }
    const float inv_a = 1.f / A;
    C[0] = cr * inv_a; C[1] = cg * inv_a; C[2] = cb * inv_a;
}

static void march_ray(const Field* F, float dt, int n_bg, float t_thresh, float w_thresh, const float o[3],
                      const float d[3], int start, float near, float mid, float far, float rgb[3], float* T_out,
                      float* depth, int32_t stats[3], int32_t* trace, int trace_cap) {
    const int n_in = mid > near ? (int)ceilf((mid - near) / dt) : 0;
    const int n_total = n_in + n_bg;
    float b[16];
    sh_basis(d[0], d[1], d[2], F->sh_deg, b);
    int cur = start, n_samples = 0, n_color = 0, walk_steps = 0;
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f}, dep = 0.f;
    for (int k = 0; k < n_total; ++k) {
        float t, delta, x[3];
        sample_at(near, mid, far, n_in, dt, n_bg, k, &t, &delta);
        for (int a = 0; a < 3; ++a) x[a] = o[a] + t * d[a];
        cur = march_walk_to(F, cur, x, &walk_steps);
        if (trace != NULL && n_samples < trace_cap) trace[n_samples] = cur;
        const float alpha = 1.f - expf(-march_density(F, cur, x) * delta);
        const float w = T * alpha;
        ++n_samples;
        if (w > w_thresh) {
            float C[3];
            march_color(F, cur, x, b, C);
            for (int a = 0; a < 3; ++a) acc[a] += w * C[a];
            dep += w * t;
            ++n_color;
        }
        T *= 1.f - alpha;
        if (T < t_thresh) break;
    }
    for (int a = 0; a < 3; ++a) rgb[a] = acc[a];
    *T_out = T;
    *depth = dep;
    stats[0] = n_samples; stats[1] = n_color; stats[2] = walk_steps;
}

double oracle_march_forward(const float* points, const int32_t* offsets, const int32_t* adj, const float* raw,
                            const float* dA, const float* cA, const float* sh, int sh_deg, const float* o,
                            const float* d, const int32_t* start, const float* near_t, const float* mid_t,
                            const float* far_t, const int64_t* rays, int64_t n_sel, float dt, int n_bg,
                            float t_thresh, float w_thresh, float* rgb, float* T, float* depth, int32_t* stats,
                            int32_t* trace, int trace_cap, int n_threads) {
    const Field F = {points, offsets, adj, raw, dA, cA, sh, sh_deg};
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
    const double t0 = omp_get_wtime();
#pragma omp parallel for schedule(dynamic, 64)
#endif
    for (int64_t i = 0; i < n_sel; ++i) {
        const int64_t r = rays != NULL ? rays[i] : i;
        march_ray(&F, dt, n_bg, t_thresh, w_thresh, o + 3 * r, d + 3 * r, start[r], near_t[r], mid_t[r], far_t[r],
                  rgb + 3 * i, T + i, depth + i, stats + 3 * i,
                  trace != NULL ? trace + (int64_t)trace_cap * i : NULL, trace_cap);
    }
#ifdef _OPENMP
    return omp_get_wtime() - t0;
#else
    return 0.0;
#endif
}

/* ==================================================================================== march_backward */

/* gA_k += gm (v v^T) in the packed symmetric layout (xx, 2xy, 2xz, yy, 2yz, zz); march.cu:86-95. */
static void add_conic_grad(float* gA, int k, float gm, const float v[3]) {
    float* a = gA + 6 * (int64_t)k;
    a[0] += gm * v[0] * v[0];
    a[1] += 2.f * gm * v[0] * v[1];
    a[2] += 2.f * gm * v[0] * v[2];
    a[3] += gm * v[1] * v[1];
    a[4] += 2.f * gm * v[1] * v[2];
    a[5] += gm * v[2] * v[2];
}

/* One ray of the backward: the forward replayed sample by sample (same walk, density, colour and stopping rule),
 * the upstream gradient of the density at each sample, d rgb / d sigma_k = delta_k (T_{k+1} C_k - (rgb - acc_k))
 * and d T / d sigma_k = -delta_k T, scattered over the sample's neighbourhood into raw and the density conic; for
 * coloured samples the gradient of C_k into the SH rows and the colour conics. march.cu:264-345 (the thresholds
 * 1e-12 on the density term and 1e-7 on the normalised colour weight are the reference's). */
static void march_ray_backward(const Field* F, float dt, int n_bg, float t_thresh, float w_thresh, const float o[3],
                               const float d[3], int start, float near, float mid, float far, const float fg[3],
                               float T_out, const float gR[3], float gT, float* g_raw, float* g_dA, float* g_cA,
                               float* g_sh) {
    const int n_in = mid > near ? (int)ceilf((mid - near) / dt) : 0;
    const int n_total = n_in + n_bg;
    const int nb = (F->sh_deg + 1) * (F->sh_deg + 1);
    float b[16];
    sh_basis(d[0], d[1], d[2], F->sh_deg, b);
    const float gT_final = gT * T_out;
    int cur = start, walk_steps = 0;
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f};
    for (int k = 0; k < n_total; ++k) {
        float t, delta, x[3];
        sample_at(near, mid, far, n_in, dt, n_bg, k, &t, &delta);
        for (int a = 0; a < 3; ++a) x[a] = o[a] + t * d[a];
        cur = march_walk_to(F, cur, x, &walk_steps);
        const float alpha = 1.f - expf(-march_density(F, cur, x) * delta);
        const float w = T * alpha;
        const float T_next = T * (1.f - alpha);
        const int active = w > w_thresh;
        float C[3] = {0.f, 0.f, 0.f}, mmin = K_INF, inv_a = 0.f;
        const int e0 = F->offsets[cur], n = F->offsets[cur + 1] - e0 + 1;
        if (active) {
            /* the colour blend of march_color, keeping m_min and 1 / sum of the shifted weights */
            for (int e = 0; e < n; ++e) {
                const int q = neighbor(F, cur, e0, e);
                const float* p = F->points + 3 * (int64_t)q;
                const float v[3] = {x[0] - p[0], x[1] - p[1], x[2] - p[2]};
                mmin = fminf(mmin, conic_maha(F->cA, q, v));
            }
            float A = 0.f, cs[3] = {0.f, 0.f, 0.f};
            for (int e = 0; e < n; ++e) {
                const int q = neighbor(F, cur, e0, e);
                const float* p = F->points + 3 * (int64_t)q;
                const float v[3] = {x[0] - p[0], x[1] - p[1], x[2] - p[2]};
                const float a = expf(-0.5f * (conic_maha(F->cA, q, v) - mmin));
                float c[3];
                sh_eval(F->sh, q, b, nb, c);
                A += a;
                for (int ch = 0; ch < 3; ++ch) cs[ch] += a * fmaxf(c[ch], 0.f);
            }
            inv_a = 1.f / A;
            for (int ch = 0; ch < 3; ++ch) C[ch] = cs[ch] * inv_a;
            for (int ch = 0; ch < 3; ++ch) acc[ch] += w * C[ch];
        }
        float gsig = 0.f;
        for (int ch = 0; ch < 3; ++ch) gsig += gR[ch] * (T_next * C[ch] - (fg[ch] - acc[ch]));
        gsig = delta * (gsig - gT_final);
        if (gsig != 0.f) {
            for (int e = 0; e < n; ++e) {
                const int q = neighbor(F, cur, e0, e);
                const float* p = F->points + 3 * (int64_t)q;
                const float v[3] = {x[0] - p[0], x[1] - p[1], x[2] - p[2]};
                const float gc = gsig * expf(fminf(F->raw[q], 30.f) - 0.5f * conic_maha(F->dA, q, v));
                if (fabsf(gc) > 1e-12f) {
                    g_raw[q] += gc;
                    add_conic_grad(g_dA, q, -0.5f * gc, v);
                }
            }
        }
        if (active) {
            const float gC[3] = {w * gR[0], w * gR[1], w * gR[2]};
            const float gCC = gC[0] * C[0] + gC[1] * C[1] + gC[2] * C[2];
            for (int e = 0; e < n; ++e) {
                const int q = neighbor(F, cur, e0, e);
                const float* p = F->points + 3 * (int64_t)q;
                const float v[3] = {x[0] - p[0], x[1] - p[1], x[2] - p[2]};
                const float a = expf(-0.5f * (conic_maha(F->cA, q, v) - mmin)) * inv_a;
                if (a < 1e-7f) continue;
                float c[3];
                sh_eval(F->sh, q, b, nb, c);
                float* gs = g_sh + 48 * (int64_t)q;
                for (int ch = 0; ch < 3; ++ch) {
                    const float dc = c[ch] > 0.f ? a * gC[ch] : 0.f;
                    for (int j = 0; j < nb; ++j) gs[3 * j + ch] += b[j] * dc;
                }
                const float ga = gC[0] * fmaxf(c[0], 0.f) + gC[1] * fmaxf(c[1], 0.f) + gC[2] * fmaxf(c[2], 0.f);
                add_conic_grad(g_cA, q, -0.5f * a * (ga - gCC), v);
            }
        }
        T = T_next;
        if (T < t_thresh) break;
    }
}

/* Gradients of a march over rays 0..B-1 (sequential, so the sums are deterministic); g_* are accumulated into
 * (the caller zeroes them). march.cu:264-345, host march_backward :402-428. */
void oracle_march_backward(const float* points, const int32_t* offsets, const int32_t* adj, const float* raw,
                           const float* dA, const float* cA, const float* sh, int sh_deg, const float* o,
                           const float* d, const int32_t* start, const float* near_t, const float* mid_t,
                           const float* far_t, int64_t B, float dt, int n_bg, float t_thresh, float w_thresh,
                           const float* rgb, const float* T, const float* g_rgb, const float* g_T, float* g_raw,
                           float* g_dA, float* g_cA, float* g_sh) {
    const Field F = {points, offsets, adj, raw, dA, cA, sh, sh_deg};
    for (int64_t r = 0; r < B; ++r)
        march_ray_backward(&F, dt, n_bg, t_thresh, w_thresh, o + 3 * r, d + 3 * r, start[r], near_t[r], mid_t[r],
                           far_t[r], rgb + 3 * r, T[r], g_rgb + 3 * r, g_T[r], g_raw, g_dA, g_cA, g_sh);
}

/* ================================================================ foam (training renderer) forward/backward */

/* A sample of the training renderer: foam.cu:272-286 (the record is t, site, sigma, C, m_min, 1 / A or 0). */
typedef struct {
    float t, x[3], sigma, C[3], mmin, inv_a;
    int site, has_c;
} TSample;

/* Exit of cell i: smallest bisector parameter ahead of the ray, ties to the smaller neighbour index;
 * foam.cu:183-206. */
static void train_exit_face(const Field* F, int i, const float o[3], const float d[3], float* t_exit, int* next) {
    const float* pi = F->points + 3 * (int64_t)i;
    float bt = K_INF;
    int bk = INT_MAX;
    for (int e = F->offsets[i]; e < F->offsets[i + 1]; ++e) {
        const int j = F->adj[e];
        const float* pj = F->points + 3 * (int64_t)j;
        float n[3], m[3];
        for (int a = 0; a < 3; ++a) {
            n[a] = pj[a] - pi[a];
            m[a] = 0.5f * (pj[a] + pi[a]) - o[a];
        }
        const float dn = n[0] * d[0] + n[1] * d[1] + n[2] * d[2];
        if (dn > 0.f) {
            const float t = (m[0] * n[0] + m[1] * n[1] + m[2] * n[2]) / dn;
            if (t < bt || (t == bt && j < bk)) { bt = t; bk = j; }
        }
    }
    *t_exit = bt;
    *next = bk;
}

/* make_sample: foam.cu:245-253. */
static void train_make(const Field* F, const float o[3], const float d[3], float t, int site, TSample* P) {
    P->t = t;
    for (int a = 0; a < 3; ++a) P->x[a] = o[a] + t * d[a];
    P->site = site;
    P->sigma = march_density(F, site, P->x);
    P->has_c = 0;
    P->inv_a = 0.f;
    P->mmin = 0.f;
    P->C[0] = P->C[1] = P->C[2] = 0.f;
}

/* color_at with m_min and 1 / A kept: foam.cu:217-243. */
static void train_color(const Field* F, TSample* P, const float b[16]) {
    const int i = P->site, e0 = F->offsets[i], n = F->offsets[i + 1] - e0 + 1;
    const int nb = (F->sh_deg + 1) * (F->sh_deg + 1);
    float mmin = K_INF;
    for (int e = 0; e < n; ++e) {
        const int k = neighbor(F, i, e0, e);
        const float* p = F->points + 3 * (int64_t)k;
        const float v[3] = {P->x[0] - p[0], P->x[1] - p[1], P->x[2] - p[2]};
        mmin = fminf(mmin, conic_maha(F->cA, k, v));
    }
    float A = 0.f, cs[3] = {0.f, 0.f, 0.f};
    for (int e = 0; e < n; ++e) {
        const int k = neighbor(F, i, e0, e);
        const float* p = F->points + 3 * (int64_t)k;
        const float v[3] = {P->x[0] - p[0], P->x[1] - p[1], P->x[2] - p[2]};
        const float a = expf(-0.5f * (conic_maha(F->cA, k, v) - mmin));
        float c[3];
        sh_eval(F->sh, k, b, nb, c);
        A += a;
        for (int ch = 0; ch < 3; ++ch) cs[ch] += a * fmaxf(c[ch], 0.f);
    }
    P->mmin = mmin;
    P->inv_a = 1.f / A;
    for (int ch = 0; ch < 3; ++ch) P->C[ch] = cs[ch] * P->inv_a;
    P->has_c = 1;
}

static void train_store(float* rec, int K, int s, const TSample* P) {
    if (rec == NULL || s >= K) return;
    float* q = rec + 8 * (int64_t)s;
    int32_t site = P->site;
    q[0] = P->t;
    memcpy(q + 1, &site, 4);
    q[2] = P->sigma;
    q[3] = P->C[0]; q[4] = P->C[1]; q[5] = P->C[2];
    q[6] = P->mmin;
    q[7] = P->has_c ? P->inv_a : 0.f;
}

/* Training forward of one ray: x(near) in the walked cell, then every exit crossing, up to x(far), trapezoid
 * compositing, colours only for segments of weight > w_thresh; foam.cu:345-393. */
static void train_ray(const Field* F, float t_thresh, float w_thresh, const float o[3], const float d[3], int start,
                     float near, float far, float rgb[3], float* T_out, float* depth, int32_t stats[3], float* rec,
                     int K) {
    float b[16];
    sh_basis(d[0], d[1], d[2], F->sh_deg, b);
    int walk_steps = 0, n_samples = 1, n_color = 0;
    float x0[3];
    for (int a = 0; a < 3; ++a) x0[a] = o[a] + near * d[a];
    int cur = march_walk_to(F, start, x0, &walk_steps);
    TSample P, Q;
    train_make(F, o, d, near, cur, &P);
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f}, dep = 0.f;
    for (int it = 0; it < K_MAX_CELLS; ++it) {
        float te;
        int nx;
        train_exit_face(F, cur, o, d, &te, &nx);
        const int last = nx == INT_MAX || te >= far;
        train_make(F, o, d, last ? far : fmaxf(te, P.t), last ? cur : nx, &Q);
        ++n_samples;
        const float delta = Q.t - P.t;
        const float alpha = 1.f - expf(-0.5f * (P.sigma + Q.sigma) * delta);
        const float w = T * alpha;
        if (w > w_thresh) {
            if (!P.has_c) train_color(F, &P, b);
            train_color(F, &Q, b);
            for (int a = 0; a < 3; ++a) acc[a] += w * 0.5f * (P.C[a] + Q.C[a]);
            dep += w * 0.5f * (P.t + Q.t);
            ++n_color;
        }
        T *= 1.f - alpha;
        train_store(rec, K, n_samples - 2, &P);
        P = Q;
        cur = Q.site;
        if (last || T < t_thresh) break;
    }
    train_store(rec, K, n_samples - 1, &P);
    for (int a = 0; a < 3; ++a) rgb[a] = acc[a];
    *T_out = T;
    *depth = dep;
    stats[0] = n_samples; stats[1] = n_color; stats[2] = walk_steps;
}

void oracle_foam_forward(const float* points, const int32_t* offsets, const int32_t* adj, const float* raw,
                         const float* dA, const float* cA, const float* sh, int sh_deg, const float* o,
                         const float* d, const int32_t* start, const float* near_t, const float* far_t, int64_t B,
                         float t_thresh, float w_thresh, float* rgb, float* T, float* depth, int32_t* stats,
                         float* rec, int K) {
    const Field F = {points, offsets, adj, raw, dA, cA, sh, sh_deg};
    for (int64_t r = 0; r < B; ++r)
        train_ray(&F, t_thresh, w_thresh, o + 3 * r, d + 3 * r, start[r], near_t[r], far_t[r], rgb + 3 * r, T + r,
                 depth + r, stats + 3 * r, rec != NULL ? rec + 8 * (int64_t)K * r : NULL, K);
}

/* A sample's gradients: gs = dL/dsigma, gC = dL/dC; foam.cu:303-343. */
static void train_scatter(const Field* F, const TSample* P, float gs, const float gC[3], const float b[16],
                         float* g_raw, float* g_dA, float* g_cA, float* g_sh) {
    const int i = P->site, e0 = F->offsets[i], n = F->offsets[i + 1] - e0 + 1;
    if (gs != 0.f) {
        for (int e = 0; e < n; ++e) {
            const int q = neighbor(F, i, e0, e);
            const float* p = F->points + 3 * (int64_t)q;
            const float v[3] = {P->x[0] - p[0], P->x[1] - p[1], P->x[2] - p[2]};
            const float gc = gs * expf(fminf(F->raw[q], 30.f) - 0.5f * conic_maha(F->dA, q, v));
            if (fabsf(gc) > 1e-12f) {
                g_raw[q] += gc;
                add_conic_grad(g_dA, q, -0.5f * gc, v);
            }
        }
    }
    if (!P->has_c || (gC[0] == 0.f && gC[1] == 0.f && gC[2] == 0.f)) return;
    const int nb = (F->sh_deg + 1) * (F->sh_deg + 1);
    const float gCC = gC[0] * P->C[0] + gC[1] * P->C[1] + gC[2] * P->C[2];
    for (int e = 0; e < n; ++e) {
        const int q = neighbor(F, i, e0, e);
        const float* p = F->points + 3 * (int64_t)q;
        const float v[3] = {P->x[0] - p[0], P->x[1] - p[1], P->x[2] - p[2]};
        const float a = expf(-0.5f * (conic_maha(F->cA, q, v) - P->mmin)) * P->inv_a;
        if (a < 1e-7f) continue;
        float c[3];
        sh_eval(F->sh, q, b, nb, c);
        float* gsh = g_sh + 48 * (int64_t)q;
        for (int ch = 0; ch < 3; ++ch) {
            const float dc = c[ch] > 0.f ? a * gC[ch] : 0.f;
            for (int j = 0; j < nb; ++j) gsh[3 * j + ch] += b[j] * dc;
        }
        const float ga = gC[0] * fmaxf(c[0], 0.f) + gC[1] * fmaxf(c[1], 0.f) + gC[2] * fmaxf(c[2], 0.f);
        const float gm = -0.5f * a * (ga - gCC);
        if (gm != 0.f) add_conic_grad(g_cA, q, gm, v);
    }
}

/* Training backward of one ray, re-tracing it (the reference's replay of recorded samples gives the same values):
 * each sample collects half of the segment gradients on both sides; foam.cu:395-469. */
static void train_ray_backward(const Field* F, float t_thresh, float w_thresh, const float o[3], const float d[3],
                              int start, float near, float far, const float fg[3], float T_out, const float gR[3],
                              float gT, float* g_raw, float* g_dA, float* g_cA, float* g_sh) {
    float b[16];
    sh_basis(d[0], d[1], d[2], F->sh_deg, b);
    const float gT_final = gT * T_out;
    int walk_steps = 0;
    float x0[3];
    for (int a = 0; a < 3; ++a) x0[a] = o[a] + near * d[a];
    int cur = march_walk_to(F, start, x0, &walk_steps);
    TSample P, Q;
    train_make(F, o, d, near, cur, &P);
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f}, gs_pending = 0.f, gC_pending[3] = {0.f, 0.f, 0.f};
    for (int it = 0; it < K_MAX_CELLS; ++it) {
        float te;
        int nx;
        train_exit_face(F, cur, o, d, &te, &nx);
        const int last = nx == INT_MAX || te >= far;
        train_make(F, o, d, last ? far : fmaxf(te, P.t), last ? cur : nx, &Q);
        const float delta = Q.t - P.t;
        const float alpha = 1.f - expf(-0.5f * (P.sigma + Q.sigma) * delta);
        const float w = T * alpha;
        const float T_next = T * (1.f - alpha);
        const int active = w > w_thresh;
        float c[3] = {0.f, 0.f, 0.f};
        if (active) {
            if (!P.has_c) train_color(F, &P, b);
            if (!Q.has_c) train_color(F, &Q, b);
            for (int a = 0; a < 3; ++a) {
                c[a] = 0.5f * (P.C[a] + Q.C[a]);
                acc[a] += w * c[a];
            }
        }
        float g_sbar = 0.f;
        for (int a = 0; a < 3; ++a) g_sbar += gR[a] * (T_next * c[a] - (fg[a] - acc[a]));
        g_sbar = delta * (g_sbar - gT_final);
        float gc_half[3], gC_P[3];
        for (int a = 0; a < 3; ++a) {
            gc_half[a] = active ? 0.5f * w * gR[a] : 0.f;
            gC_P[a] = gC_pending[a] + gc_half[a];
        }
        train_scatter(F, &P, gs_pending + 0.5f * g_sbar, gC_P, b, g_raw, g_dA, g_cA, g_sh);
        gs_pending = 0.5f * g_sbar;
        for (int a = 0; a < 3; ++a) gC_pending[a] = gc_half[a];
        T = T_next;
        P = Q;
        cur = Q.site;
        if (last || T < t_thresh) break;
    }
    train_scatter(F, &P, gs_pending, gC_pending, b, g_raw, g_dA, g_cA, g_sh);
}

void oracle_foam_backward(const float* points, const int32_t* offsets, const int32_t* adj, const float* raw,
                          const float* dA, const float* cA, const float* sh, int sh_deg, const float* o,
                          const float* d, const int32_t* start, const float* near_t, const float* far_t, int64_t B,
                          float t_thresh, float w_thresh, const float* rgb, const float* T, const float* g_rgb,
                          const float* g_T, float* g_raw, float* g_dA, float* g_cA, float* g_sh) {
    const Field F = {points, offsets, adj, raw, dA, cA, sh, sh_deg};
    for (int64_t r = 0; r < B; ++r)
        train_ray_backward(&F, t_thresh, w_thresh, o + 3 * r, d + 3 * r, start[r], near_t[r], far_t[r], rgb + 3 * r,
                          T[r], g_rgb + 3 * r, g_T[r], g_raw, g_dA, g_cA, g_sh);
}

/* ============================================================================ vgf forward operators */

/* Greedy walk of S sorted samples per ray, strict < (first found wins), starting at the previous site;
 * vgf.cu:44-79. */
void oracle_walk(const float* points, const int32_t* offsets, const int32_t* adj, const float* o, const float* d,
                 const float* z, const int32_t* start, int64_t B, int S, int32_t* site, int32_t* steps, int n_threads) {
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#pragma omp parallel for schedule(dynamic, 64)
#endif
    for (int64_t r = 0; r < B; ++r) {
        const float ox = o[3 * r], oy = o[3 * r + 1], oz = o[3 * r + 2];
        const float dx = d[3 * r], dy = d[3 * r + 1], dz = d[3 * r + 2];
        int cur = start[r], total = 0;
        for (int s = 0; s < S; ++s) {
            const float t = z[r * S + s];
            const float x = ox + t * dx, y = oy + t * dy, w = oz + t * dz;
            const float* pc = points + 3 * (int64_t)cur;
            const float cx = x - pc[0], cy = y - pc[1], cz = w - pc[2];
            float best_d = cx * cx + cy * cy + cz * cz;
            for (int it = 0; it < K_WALK_CAP; ++it) {
                int best = cur;
                const int e1 = offsets[cur + 1];
                for (int e = offsets[cur]; e < e1; ++e) {
                    const int q = adj[e];
                    const float* p = points + 3 * (int64_t)q;
                    const float qx = x - p[0], qy = y - p[1], qz = w - p[2];
                    const float dq = qx * qx + qy * qy + qz * qz;
                    if (dq < best_d) { best_d = dq; best = q; }
                }
                if (best == cur) break;
                cur = best;
                ++total;
            }
            site[r * S + s] = cur;
        }
        if (steps != NULL) steps[r] = total;
    }
}

/* Mahalanobis distance of x to Gaussian i from (log_scale, quat), with 1/s^2 scaled by inv_mult2;
 * vgf.cu:98-119. */
static float gauss_m(const float* points, const float* log_scale, const float* quat, int i, float x, float y, float z,
                     float inv_mult2) {
    const int64_t i3 = 3 * (int64_t)i;
    const float v0 = x - points[i3], v1 = y - points[i3 + 1], v2 = z - points[i3 + 2];
    const float* q = quat + 4 * (int64_t)i;
    const float qnorm = fmaxf(sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]), 1e-12f);
    const float w = q[0] / qnorm, a = q[1] / qnorm, b = q[2] / qnorm, c = q[3] / qnorm;
    float R[9];
    R[0] = 1.f - 2.f * (b * b + c * c); R[1] = 2.f * (a * b - w * c); R[2] = 2.f * (a * c + w * b);
    R[3] = 2.f * (a * b + w * c); R[4] = 1.f - 2.f * (a * a + c * c); R[5] = 2.f * (b * c - w * a);
    R[6] = 2.f * (a * c - w * b); R[7] = 2.f * (b * c + w * a); R[8] = 1.f - 2.f * (a * a + b * b);
    float m = 0.f;
    for (int k = 0; k < 3; ++k) {
        const float yk = R[k] * v0 + R[3 + k] * v1 + R[6 + k] * v2;
        const float s = expf(fminf(fmaxf(log_scale[i3 + k], -20.f), 20.f));
        const float is2 = inv_mult2 / (s * s);
        m += yk * yk * is2;
    }
    return m;
}

/* sigma(x) = sum over {i} U adj(i) of exp(min(raw_k, 30) - m_k / 2); vgf.cu:152-177. */
void oracle_density(const float* points, const int32_t* offsets, const int32_t* adj, const float* raw,
                    const float* log_scale, const float* quat, const float* x, const int32_t* site, int64_t m,
                    float scale_mult, float* sigma, int n_threads) {
    const float inv_mult2 = (float)(1.0 / ((double)scale_mult * (double)scale_mult));
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#pragma omp parallel for schedule(static)
#endif
    for (int64_t t = 0; t < m; ++t) {
        const float qx = x[3 * t], qy = x[3 * t + 1], qz = x[3 * t + 2];
        const int i = site[t];
        float s = 0.f;
        for (int e = offsets[i] - 1; e < offsets[i + 1]; ++e) {
            const int k = e < offsets[i] ? i : adj[e];
            s += expf(fminf(raw[k], 30.f) - 0.5f * gauss_m(points, log_scale, quat, k, qx, qy, qz, inv_mult2));
        }
        sigma[t] = s;
    }
}

/* Online-softmax blend of max(SH_k(d) + 1/2, 0) over {i} U adj(i); vgf.cu:230-282. */
void oracle_color(const float* points, const int32_t* offsets, const int32_t* adj, const float* log_scale,
                  const float* quat, const float* sh, int sh_deg, const float* x, const float* dirs,
                  const int32_t* site, int64_t m, float* rgb, int n_threads) {
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#pragma omp parallel for schedule(static)
#endif
    for (int64_t t = 0; t < m; ++t) {
        const float qx = x[3 * t], qy = x[3 * t + 1], qz = x[3 * t + 2];
        float dx = dirs[3 * t], dy = dirs[3 * t + 1], dz = dirs[3 * t + 2];
        const float inv = 1.f / sqrtf(fmaxf(dx * dx + dy * dy + dz * dz, 1e-20f));
        dx *= inv; dy *= inv; dz *= inv;
        float b[16];
        sh_basis(dx, dy, dz, sh_deg, b);
        const int nb = (sh_deg + 1) * (sh_deg + 1);
        const int i = site[t];
        float mmin = K_INF, A = 0.f, cr = 0.f, cg = 0.f, cb = 0.f;
        for (int e = offsets[i] - 1; e < offsets[i + 1]; ++e) {
            const int k = e < offsets[i] ? i : adj[e];
            const float mk = gauss_m(points, log_scale, quat, k, qx, qy, qz, 1.f);
            if (mk < mmin) {
                const float f = mmin == K_INF ? 0.f : expf(-0.5f * (mmin - mk));
                A *= f; cr *= f; cg *= f; cb *= f;
                mmin = mk;
            }
            const float a = expf(-0.5f * (mk - mmin));
            float c[3];
            sh_eval(sh, k, b, nb, c);
            A += a;
            cr += a * fmaxf(c[0], 0.f);
            cg += a * fmaxf(c[1], 0.f);
            cb += a * fmaxf(c[2], 0.f);
        }
        rgb[3 * t] = cr / A;
        rgb[3 * t + 1] = cg / A;
        rgb[3 * t + 2] = cb / A;
    }
}

/* A = R diag(1 / (s^2 + floor^2)) R^T as (xx, xy, xz, yy, yz, zz); vgf.cu:340-380. */
void oracle_conic(const float* log_scale, const float* quat, int64_t n, float floor2, float* A) {
    static const int ab[6][2] = {{0, 0}, {0, 1}, {0, 2}, {1, 1}, {1, 2}, {2, 2}};
    for (int64_t i = 0; i < n; ++i) {
        const float* q = quat + 4 * i;
        const float qnorm = fmaxf(sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]), 1e-12f);
        const float w = q[0] / qnorm, a = q[1] / qnorm, b = q[2] / qnorm, c = q[3] / qnorm;
        float R[9], iv[3];
        R[0] = 1.f - 2.f * (b * b + c * c); R[1] = 2.f * (a * b - w * c); R[2] = 2.f * (a * c + w * b);
        R[3] = 2.f * (a * b + w * c); R[4] = 1.f - 2.f * (a * a + c * c); R[5] = 2.f * (b * c - w * a);
        R[6] = 2.f * (a * c - w * b); R[7] = 2.f * (b * c + w * a); R[8] = 1.f - 2.f * (a * a + b * b);
        for (int k = 0; k < 3; ++k) {
            const float s = expf(2.f * fminf(fmaxf(log_scale[3 * i + k], -20.f), 20.f));
            iv[k] = 1.f / (s + floor2);
        }
        for (int e = 0; e < 6; ++e) {
            const int x = ab[e][0], y = ab[e][1];
            A[6 * i + e] = R[3 * x] * R[3 * y] * iv[0] + R[3 * x + 1] * R[3 * y + 1] * iv[1] +
                           R[3 * x + 2] * R[3 * y + 2] * iv[2];
        }
    }
}

/* ============================================================================ vgf backward operators */

/* Gaussian i seen from x: offset v = x - p_i, normalised quaternion qn (and the norm it was divided by), rotation
 * R (row-major, columns = the Gaussian's axes), y = R^T v, inverse variances is2 and m = sum_k y_k^2 is2_k;
 * vgf.cu:87-119 (gauss_local). */
typedef struct {
    float v[3], y[3], is2[3], qn[4], qnorm, R[9], m;
} GFrame;

static void gauss_frame(const float* points, const float* log_scale, const float* quat, int i, float x, float y,
                        float z, GFrame* L) {
    const int64_t i3 = 3 * (int64_t)i;
    L->v[0] = x - points[i3];
    L->v[1] = y - points[i3 + 1];
    L->v[2] = z - points[i3 + 2];
    const float* q = quat + 4 * (int64_t)i;
    L->qnorm = fmaxf(sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]), 1e-12f);
    for (int k = 0; k < 4; ++k) L->qn[k] = q[k] / L->qnorm;
    const float w = L->qn[0], a = L->qn[1], b = L->qn[2], c = L->qn[3];
    float* R = L->R;
    R[0] = 1.f - 2.f * (b * b + c * c); R[1] = 2.f * (a * b - w * c); R[2] = 2.f * (a * c + w * b);
    R[3] = 2.f * (a * b + w * c); R[4] = 1.f - 2.f * (a * a + c * c); R[5] = 2.f * (b * c - w * a);
    R[6] = 2.f * (a * c - w * b); R[7] = 2.f * (b * c + w * a); R[8] = 1.f - 2.f * (a * a + b * b);
    L->m = 0.f;
    for (int k = 0; k < 3; ++k) {
        L->y[k] = R[k] * L->v[0] + R[3 + k] * L->v[1] + R[6 + k] * L->v[2];
        const float s = expf(fminf(fmaxf(log_scale[i3 + k], -20.f), 20.f));
        L->is2[k] = 1.f / (s * s);
        L->m += L->y[k] * L->y[k] * L->is2[k];
    }
}

/* dL/dquat of a unit-quaternion rotation from dL/dR (row-major), through the normalisation q / |q|: the product
 * rule on R(qn) above, then the tangent projection (dq - (dq . qn) qn) / |q|; vgf.cu:132-147 and :412-423. */
static void quat_grad(const float qn[4], float qnorm, const float dR[9], float out[4]) {
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
    for (int k = 0; k < 4; ++k) out[k] = (dq[k] - proj * qn[k]) / qnorm;
}

/* Adds dL/dlog_scale and dL/dquat of Gaussian i given gm = dL/dm; vgf.cu:121-148 (scatter_gauss_grad). With
 * m = sum_k y_k^2 / s_k^2: dm/dlog_s_k = -2 y_k^2 is2_k, dm/dy_k = 2 y_k is2_k, and dy_b/dR_ab = v_a. */
static void gauss_grad(const GFrame* L, float gm, int i, float* g_ls, float* g_quat) {
    float yk[3], dR[9], gq[4];
    for (int k = 0; k < 3; ++k) {
        yk[k] = 2.f * gm * L->y[k] * L->is2[k];
        g_ls[3 * (int64_t)i + k] += -2.f * gm * L->y[k] * L->y[k] * L->is2[k];
    }
    for (int a = 0; a < 3; ++a)
        for (int b = 0; b < 3; ++b) dR[3 * a + b] = L->v[a] * yk[b];
    quat_grad(L->qn, L->qnorm, dR, gq);
    for (int k = 0; k < 4; ++k) g_quat[4 * (int64_t)i + k] += gq[k];
}

/* Gradients of oracle_density (scale_mult 1) for dL/dsigma = grad_sigma, accumulated into g_raw (N), g_ls (N, 3),
 * g_quat (N, 4) in sample order; terms with rho_k G_k |dL/dsigma| <= 1e-12 are skipped; vgf.cu:179-198. */
void oracle_density_backward(const float* points, const int32_t* offsets, const int32_t* adj, const float* raw,
                             const float* log_scale, const float* quat, const float* x, const int32_t* site, int64_t m,
                             const float* grad_sigma, float* g_raw, float* g_ls, float* g_quat) {
    for (int64_t t = 0; t < m; ++t) {
        const float gs = grad_sigma[t];
        if (gs == 0.f) continue;
        const int i = site[t];
        for (int e = offsets[i] - 1; e < offsets[i + 1]; ++e) {
            const int k = e < offsets[i] ? i : adj[e];
            GFrame L;
            gauss_frame(points, log_scale, quat, k, x[3 * t], x[3 * t + 1], x[3 * t + 2], &L);
            const float c = expf(fminf(raw[k], 30.f) - 0.5f * L.m);
            if (c * fabsf(gs) > 1e-12f) {
                g_raw[k] += gs * c;
                gauss_grad(&L, -0.5f * gs * c, k, g_ls, g_quat);
            }
        }
    }
}

/* Gradients of oracle_color for dL/drgb = grad_rgb given the forward rgb, accumulated into g_ls, g_quat and g_sh
 * (N, 16, 3) in sample order; vgf.cu:284-333. With a_k the normalised weights and C = sum a_k c_k:
 * dL/dc_k = a_k dL/dC (where SH_k + 1/2 > 0), dL/dm_k = -a_k / 2 (<dL/dC, c_k> - <dL/dC, C>); weights below 1e-7
 * get no gradient. */
void oracle_color_backward(const float* points, const int32_t* offsets, const int32_t* adj, const float* log_scale,
                           const float* quat, const float* sh, int sh_deg, const float* x, const float* dirs,
                           const int32_t* site, int64_t m, const float* rgb, const float* grad_rgb, float* g_ls,
                           float* g_quat, float* g_sh) {
    for (int64_t t = 0; t < m; ++t) {
        const float gr = grad_rgb[3 * t], gg = grad_rgb[3 * t + 1], gb = grad_rgb[3 * t + 2];
        if (gr == 0.f && gg == 0.f && gb == 0.f) continue;
        const float qx = x[3 * t], qy = x[3 * t + 1], qz = x[3 * t + 2];
        const int i = site[t];
        float mmin = K_INF, A = 0.f;
        for (int e = offsets[i] - 1; e < offsets[i + 1]; ++e) {
            const int k = e < offsets[i] ? i : adj[e];
            mmin = fminf(mmin, gauss_m(points, log_scale, quat, k, qx, qy, qz, 1.f));
        }
        for (int e = offsets[i] - 1; e < offsets[i + 1]; ++e) {
            const int k = e < offsets[i] ? i : adj[e];
            A += expf(-0.5f * (gauss_m(points, log_scale, quat, k, qx, qy, qz, 1.f) - mmin));
        }
        const float inv_a = 1.f / A;
        const float gCC = gr * rgb[3 * t] + gg * rgb[3 * t + 1] + gb * rgb[3 * t + 2];
        float dx = dirs[3 * t], dy = dirs[3 * t + 1], dz = dirs[3 * t + 2];
        const float inv = 1.f / sqrtf(fmaxf(dx * dx + dy * dy + dz * dz, 1e-20f));
        dx *= inv; dy *= inv; dz *= inv;
        float b[16];
        sh_basis(dx, dy, dz, sh_deg, b);
        const int nb = (sh_deg + 1) * (sh_deg + 1);
        for (int e = offsets[i] - 1; e < offsets[i + 1]; ++e) {
            const int k = e < offsets[i] ? i : adj[e];
            GFrame L;
            gauss_frame(points, log_scale, quat, k, qx, qy, qz, &L);
            const float a = expf(-0.5f * (L.m - mmin)) * inv_a;
            if (a < 1e-7f) continue;
            float c[3];
            sh_eval(sh, k, b, nb, c);
            const float dc[3] = {c[0] > 0.f ? a * gr : 0.f, c[1] > 0.f ? a * gg : 0.f, c[2] > 0.f ? a * gb : 0.f};
            float* gs = g_sh + 48 * (int64_t)k;
            for (int j = 0; j < nb; ++j)
                for (int ch = 0; ch < 3; ++ch) gs[3 * j + ch] += b[j] * dc[ch];
            const float ga = gr * fmaxf(c[0], 0.f) + gg * fmaxf(c[1], 0.f) + gb * fmaxf(c[2], 0.f);
            const float gm = -0.5f * a * (ga - gCC);
            if (gm != 0.f) gauss_grad(&L, gm, k, g_ls, g_quat);
        }
    }
}

/* Gradients of oracle_conic for dL/dA = gA (N, 6), written to g_ls (N, 3) and g_quat (N, 4); vgf.cu:382-424. The
 * off-diagonal entries of A stand for both A_ab and A_ba, so dL/dA is the symmetric G with G_ab = gA_ab / 2 off the
 * diagonal; with A = R diag(iv) R^T: dL/div_k = (R^T G R)_kk, div_k/dlog_s_k = -2 s_k^2 iv_k^2, dL/dR = 2 G R
 * diag(iv). */
void oracle_conic_backward(const float* log_scale, const float* quat, int64_t n, float floor2, const float* gA,
                           float* g_ls, float* g_quat) {
    for (int64_t i = 0; i < n; ++i) {
        const float* q = quat + 4 * i;
        const float qnorm = fmaxf(sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]), 1e-12f);
        float qn[4], R[9], iv[3], s2[3];
        for (int k = 0; k < 4; ++k) qn[k] = q[k] / qnorm;
        const float w = qn[0], a = qn[1], b = qn[2], c = qn[3];
        R[0] = 1.f - 2.f * (b * b + c * c); R[1] = 2.f * (a * b - w * c); R[2] = 2.f * (a * c + w * b);
        R[3] = 2.f * (a * b + w * c); R[4] = 1.f - 2.f * (a * a + c * c); R[5] = 2.f * (b * c - w * a);
        R[6] = 2.f * (a * c - w * b); R[7] = 2.f * (b * c + w * a); R[8] = 1.f - 2.f * (a * a + b * b);
        for (int k = 0; k < 3; ++k) {
            s2[k] = expf(2.f * fminf(fmaxf(log_scale[3 * i + k], -20.f), 20.f));
            iv[k] = 1.f / (s2[k] + floor2);
        }
        const float* g = gA + 6 * i;
        const float G[9] = {g[0], 0.5f * g[1], 0.5f * g[2], 0.5f * g[1], g[3], 0.5f * g[4], 0.5f * g[2], 0.5f * g[4],
                            g[5]};
        float GR[9], dR[9];
        for (int r = 0; r < 3; ++r)
            for (int k = 0; k < 3; ++k)
                GR[3 * r + k] = G[3 * r] * R[k] + G[3 * r + 1] * R[3 + k] + G[3 * r + 2] * R[6 + k];
        for (int k = 0; k < 3; ++k) {
            const float g_iv = R[k] * GR[k] + R[3 + k] * GR[3 + k] + R[6 + k] * GR[6 + k];
            g_ls[3 * i + k] = g_iv * (-2.f * s2[k] * iv[k] * iv[k]);
        }
        for (int r = 0; r < 3; ++r)
            for (int k = 0; k < 3; ++k) dR[3 * r + k] = 2.f * GR[3 * r + k] * iv[k];
        quat_grad(qn, qnorm, dR, g_quat + 4 * i);
    }
}

int oracle_omp_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
