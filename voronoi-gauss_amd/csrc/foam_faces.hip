// Cell traversal with one group of lanes per ray (lane-per-face layout), gfx950: the layout comparison for the
// inference renderer's traversal.
//
// foam_infer.hip runs one ray per lane. The other layout for wave64 tests a cell's faces in parallel: a group of
// G lanes (4, 8 or 16) serves one ray, 64 / G rays per wave; lane g of the group takes edges e0 + 1 + g,
// e0 + 1 + g + G, ... of the cell's neighbourhood, and the exit face is a group min-reduction of (t, tie order).
// The greedy walk to the start cell is a group argmin of (distance, tie order) in the same way. This kernel
// covers the traversal alone (stage 0 of foam_infer: walk, then exit faces from cell to cell up to far or `cap`
// samples; with no density T stays 1, so t_thresh <= 1 never stops a ray): the same visited cells, the same
// sample counts and walk steps, bit for bit, since a lexicographic minimum does not depend on the order in which
// it is reduced. Semantics: csrc/foam_infer.cu:176-194 (walk_to) and :199-257 (eval_cell, exit faces) of the
// reference.
//
// The reduction runs on DPP row permutations (a VALU move each, no LDS): xor 1 and xor 2 within a quad, then the
// half-row mirror (lane i <-> 7 - i) and the row mirror (i <-> 15 - i). After the steps up to width G every lane
// of the group holds the group minimum, and no step reads outside the group, so groups whose ray has finished
// (inactive lanes) are never read. Exact ties in t, which the tie order settles, are rare: they take a
// wave-uniform slow path, so the common path has no per-lane branches.
#include "vgr_abi.h"
#include "vgr_device.h"

namespace vgr {
namespace {

constexpr int kFacesBlock = 64;  // one wave per workgroup

struct FacesScene {
    const float4* __restrict__ points;  // (N) p, w unused
    const int* __restrict__ offsets;    // (N + 1) self-first
    const int* __restrict__ nbr;        // (E)
    const float4* __restrict__ edge;    // (E) p_j, cut-off word
    const int* __restrict__ orig;       // (N) or null
    int n_sites;
};

// k precedes j in the tie order: the smaller original index (INT_MAX: no site, after every site).
__device__ __noinline__ bool before_site(const FacesScene& S, int k, int j) {
    if (j == INT_MAX) return k != INT_MAX;
    if (k == INT_MAX) return false;
    return S.orig != nullptr ? S.orig[k] < S.orig[j] : k < j;
}

__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// Keeps the lexicographic minimum of (t, k) and the candidate (u, j): strict `<` on t, the tie order on equal t.
__device__ __forceinline__ void keep_min(const FacesScene& S, float u, int j, float& t, int& k) {
    bool take = u < t;
    const bool tie = u == t && j != k;
    if (wave_any(tie)) {  // wave-uniform branch; inside, only the tied lanes look up the tie order
        if (tie) take = before_site(S, j, k);
    }
    if (take) t = u, k = j;
}

template <int CTRL>
__device__ __forceinline__ void reduce_step(const FacesScene& S, float& t, int& k) {
    const float u = row_perm<CTRL>(t);
    const int j = row_perm<CTRL>(k);
    keep_min(S, u, j, t, k);
}

// Group-wide lexicographic minimum of (t, k) over the G lanes of the group: every lane ends with it.
template <int G>
__device__ __forceinline__ void group_min(const FacesScene& S, float& t, int& k) {
    static_assert(G == 4 || G == 8 || G == 16, "group width");
    reduce_step<kXor1>(S, t, k);
    reduce_step<kXor2>(S, t, k);
    if constexpr (G >= 8) reduce_step<kHalfMirror>(S, t, k);
    if constexpr (G >= 16) reduce_step<kMirror>(S, t, k);
}

template <int G, bool TRACE>
__global__ void __launch_bounds__(kFacesBlock)
    foam_faces_kernel(FacesScene S, const float* __restrict__ o_, const float* __restrict__ d_,
                      const int* __restrict__ start_, const float* __restrict__ near_, const float* __restrict__ far_,
                      const int* __restrict__ cap, int64_t n_rays, int* __restrict__ stats, int* __restrict__ trace,
                      int64_t trace_cap) {
    constexpr int kRaysPerBlock = kFacesBlock / G;
    const int g = static_cast<int>(threadIdx.x) % G;
    const int64_t r = xcd_block_id() * kRaysPerBlock + threadIdx.x / G;
    if (r >= n_rays) return;  // whole groups leave together: every reduction stays within a live group
    int* st = stats + 5 * r;
    int cur = start_[r];
    if (cur < 0 || cur >= S.n_sites) {  // not traced
        if (g == 0) st[0] = st[1] = st[2] = st[3] = st[4] = 0;
        return;
    }
    const float o[3] = {o_[3 * r], o_[3 * r + 1], o_[3 * r + 2]};
    const float d[3] = {d_[3 * r], d_[3 * r + 1], d_[3 * r + 2]};
    const float t_near = near_[r], t_far = far_[r];
    const int max_samples = cap != nullptr ? cap[r] : INT_MAX;

    // greedy walk to the cell of x(near): the group argmin over {c} U adj(c), repeated until c wins
    int walk_steps = 0;
    {
        const float x0 = o[0] + t_near * d[0], x1 = o[1] + t_near * d[1], x2 = o[2] + t_near * d[2];
        for (int it = 0; it < kWalkCap; ++it) {
            const float4 pc = S.points[cur];
            float bd = (x0 - pc.x) * (x0 - pc.x) + (x1 - pc.y) * (x1 - pc.y) + (x2 - pc.z) * (x2 - pc.z);
            int bk = cur;
            const int e0 = S.offsets[cur], e1 = S.offsets[cur + 1];
            for (int e = e0 + 1 + g; e < e1; e += G) {
                const float4 ed = S.edge[e];
                const int k = S.nbr[e];
                const float v0 = x0 - ed.x, v1 = x1 - ed.y, v2 = x2 - ed.z;
                keep_min(S, v0 * v0 + v1 * v1 + v2 * v2, k, bd, bk);
            }
            group_min<G>(S, bd, bk);
            if (bk == cur) break;
            cur = bk;
            ++walk_steps;
        }
    }

    // the exit face of cell c: group minimum of the bisector-plane parameters of the faces ahead (n . d > 0)
    auto face_t = [&](const float4& pc, const float4& ed, bool& ahead) {
        const float n0 = ed.x - pc.x, n1 = ed.y - pc.y, n2 = ed.z - pc.z;
        const float dn = n0 * d[0] + n1 * d[1] + n2 * d[2];
        const float m0 = 0.5f * (ed.x + pc.x) - o[0], m1 = 0.5f * (ed.y + pc.y) - o[1],
                    m2 = 0.5f * (ed.z + pc.z) - o[2];
        ahead = dn > 0.f;
        return (m0 * n0 + m1 * n1 + m2 * n2) / dn;
    };
    auto exit_face = [&](int c, float& t_exit, int& next) {
        const float4 pc = S.points[c];
        t_exit = kInf, next = INT_MAX;
        const int e0 = S.offsets[c], e1 = S.offsets[c + 1];
        for (int e = e0 + 1 + g; e < e1; e += 2 * G) {  // two faces per lane per trip, both loads issued first
            const bool second = e + G < e1;
            const float4 ea = S.edge[e];
            const int ka = S.nbr[e];
            float4 eb = ea;
            int kb = INT_MAX;
            if (second) eb = S.edge[e + G], kb = S.nbr[e + G];
            bool ahead_a, ahead_b;
            const float ta = face_t(pc, ea, ahead_a);
            if (ahead_a) keep_min(S, ta, ka, t_exit, next);
            const float tb = face_t(pc, eb, ahead_b);
            if (second && ahead_b) keep_min(S, tb, kb, t_exit, next);
        }
        group_min<G>(S, t_exit, next);
    };

    if (TRACE && g == 0 && trace_cap > 0) trace[r * trace_cap] = S.orig != nullptr ? S.orig[cur] : cur;
    float t_exit;
    int next;
    exit_face(cur, t_exit, next);
    float tP = t_near;
    int n_samples = 1;
    for (int it = 0; it < kMaxCells; ++it) {
        const bool last = next == INT_MAX || t_exit >= t_far || n_samples + 1 >= max_samples;
        const float tQ = last ? t_far : fmaxf(t_exit, tP);
        if (!last) cur = next;
        if (TRACE && g == 0 && n_samples < trace_cap)
            trace[r * trace_cap + n_samples] = S.orig != nullptr ? S.orig[cur] : cur;
        ++n_samples;
        if (last) break;
        exit_face(cur, t_exit, next);
        tP = tQ;
    }
    if (g == 0) st[0] = n_samples, st[1] = 0, st[2] = walk_steps, st[3] = 0, st[4] = 0;
}

template <int G>
void launch_faces(const FacesScene& S, const float* o, const float* d, const int32_t* start, const float* near_t,
                  const float* far_t, int64_t n_rays, const int32_t* cap, int32_t* stats, int32_t* trace,
                  int64_t trace_cap, hipStream_t stream) {
    const dim3 grid(grid_for(n_rays, kFacesBlock / G)), block(kFacesBlock);
    if (trace != nullptr)
        hipLaunchKernelGGL((foam_faces_kernel<G, true>), grid, block, 0, stream, S, o, d, start, near_t, far_t, cap,
                           n_rays, stats, trace, trace_cap);
    else
        hipLaunchKernelGGL((foam_faces_kernel<G, false>), grid, block, 0, stream, S, o, d, start, near_t, far_t, cap,
                           n_rays, stats, trace, int64_t{0});
}

}  // namespace
}  // namespace vgr

extern "C" int vgr_foam_traverse_faces(const float* points, int64_t n_sites, const int32_t* offsets,
                                       const int32_t* nbr, const float* edge, int64_t n_edges, const float* o,
                                       const float* d, const int32_t* start, const float* near_t, const float* far_t,
                                       int64_t n_rays, const int32_t* cap, const int32_t* orig, int32_t* stats,
                                       int32_t* trace, int64_t trace_cap, int64_t lanes_per_ray, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(n_rays >= 0, "foam_traverse_faces: n_rays must be >= 0");
    VGR_REQUIRE(trace == nullptr || trace_cap > 0, "foam_traverse_faces: trace needs trace_cap > 0");
    VGR_REQUIRE(lanes_per_ray == 0 || lanes_per_ray == 4 || lanes_per_ray == 8 || lanes_per_ray == 16,
                "foam_traverse_faces: lanes_per_ray must be 4, 8 or 16 (0: the default, 4)");
    if (n_rays == 0) return VGR_OK;
    VGR_REQUIRE(n_sites > 0 && n_sites <= INT_MAX, "foam_traverse_faces: n_sites must be in [1, 2^31)");
    VGR_REQUIRE(n_edges >= n_sites && n_edges <= INT_MAX, "foam_traverse_faces: n_edges must be in [N, 2^31)");
    VGR_REQUIRE(points && offsets && nbr && edge, "foam_traverse_faces: null scene pointer");
    VGR_REQUIRE(o && d && start && near_t && far_t && stats, "foam_traverse_faces: null ray pointer");
    const FacesScene S{reinterpret_cast<const float4*>(points), offsets, nbr, reinterpret_cast<const float4*>(edge),
                       orig, int(n_sites)};
    const hipStream_t s = as_stream(stream);
    switch (lanes_per_ray) {
        case 8: launch_faces<8>(S, o, d, start, near_t, far_t, n_rays, cap, stats, trace, trace_cap, s); break;
        case 16: launch_faces<16>(S, o, d, start, near_t, far_t, n_rays, cap, stats, trace, trace_cap, s); break;
        default: launch_faces<4>(S, o, d, start, near_t, far_t, n_rays, cap, stats, trace, trace_cap, s); break;
    }
    return launch_status("foam_faces_kernel");
}
