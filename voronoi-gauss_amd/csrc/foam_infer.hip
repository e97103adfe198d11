// Inference renderer at the ray / Voronoi-face interaction points, gfx950.
//
// Semantics follow csrc/foam_infer.cu:50-361 of the reference: a ray starts in the cell of x(near) (greedy
// walk from `start`), then crosses cells through their exit faces (the nearest bisector plane ahead of the
// ray); every crossing is a sample evaluated with the self-first neighbourhood of the cell it enters, and
// consecutive samples are composited with the trapezoid rule until x(far), `cap` samples, or T < t_thresh.
//
// MI355X mapping: one ray per lane, rays ordered in 8x8 pixel tiles by the host so a wave64 is one tile and
// its lanes walk mostly the same cells (the per-edge loads of a cell are then one broadcast line per wave);
// workgroups are remapped so each XCD renders a contiguous band of tiles (L2 locality). SH coefficient blocks
// are cached per wave in LDS (the tile's rays read mostly the same sites); colours are evaluated per lane.
// A second layout, a group of 2, 4 or 8 lanes per ray (foam_group_kernel below), splits each cell's
// neighbourhood over the group's lanes; it is the faster one for traversal, density and lazy colours, one ray per
// lane for fused and baked colours (default_lanes).
#include <cmath>
#include <type_traits>

#include "vgr_abi.h"
#include "vgr_device.h"

namespace vgr {
namespace {

constexpr int kBlock = 64;  // one wave64 per workgroup = one 8x8 ray tile
constexpr int kLazy = VGR_COLOR_LAZY, kBaked = VGR_COLOR_BAKED, kFused = VGR_COLOR_FUSED;
// Fused colours over the indexed edge records (vgr_foam_index_pack): the neighbour's index in the fourth word of its
// edge record and its cut-off word in attr[:, 7], so a neighbour round loads no separate index. An internal mode of
// this file: it blends exactly as kFused.
constexpr int kFusedIdx = 3;

struct FoamScene {
    const float4* __restrict__ points;  // (N) p, w unused
    const int* __restrict__ offsets;    // (N + 1) self-first
    const int* __restrict__ nbr;        // (E)
    const float4* __restrict__ edge;    // (E) p_j, half2(r2_j, lam_j)
    const float4* __restrict__ attr;    // (N, 5)
    const float4* __restrict__ sh;      // (N, 12) fp32 or (N, 6) fp16
    const int* __restrict__ orig;       // (N) or null
    const int4* __restrict__ slots;     // (N, 4) slot table (vgr_foam_slot_table) or null
    const float4* __restrict__ rows;    // site rows (the first 16 attr columns) or null, row_stride float4 apart
    int n_sites;
    int row_stride;  // float4 from one site row to the next: 4 (64-byte rows) or 16 (256-byte site blocks)
    int sh_stride;   // float4 from one SH row to the next: 12 (fp32), 6 (fp16) or 16 (the SH rows of site blocks)
};

struct FoamParams {
    float t_thresh, w_thresh, color_cut;
    int sh_deg;
};

struct FoamRays {
    const float* __restrict__ o;
    const float* __restrict__ d;
    const int* __restrict__ start;
    const float* __restrict__ t_near;
    const float* __restrict__ t_far;
    const int* __restrict__ cap;
    int64_t n;
    const int* __restrict__ order;  // processing order of the rays (a permutation of 0 .. n - 1), or null
};

struct FoamOut {
    float* __restrict__ rgb;
    float* __restrict__ T;
    float* __restrict__ depth;
    int* __restrict__ stats;
    int* __restrict__ trace;
    int64_t trace_cap;
};

// Running normalised colour blend (fused / baked modes).
struct Blend {
    float m, a, r, g, b;
};

__device__ __forceinline__ void blend_init(Blend& B) { B.m = kInf, B.a = B.r = B.g = B.b = 0.f; }

// k precedes j in the tie-breaking order: the smaller original index.
__device__ __forceinline__ bool before(const FoamScene& S, int k, int j) {
    return S.orig != nullptr ? S.orig[k] < S.orig[j] : k < j;
}

// (r2, lam) half2 packed in the 4th component of an edge record.
__device__ __forceinline__ float2 cutoffs(float w) {
    const uint32_t u = __float_as_uint(w);
    const _Float16 lo = __builtin_bit_cast(_Float16, static_cast<uint16_t>(u & 0xffffu));
    const _Float16 hi = __builtin_bit_cast(_Float16, static_cast<uint16_t>(u >> 16));
    return make_float2(static_cast<float>(lo), static_cast<float>(hi));
}

// ------------------------------------------------------------------ field arithmetic (explicit FMA)
// The density, colour and blend arithmetic below fuses chosen products and sums into one FMA (fmaf), which rounds
// once where the CPU oracle rounds twice: each term moves by at most an ulp of its magnitude, and the colours and
// transmittances by a few ulps of 1 (about 1e-6), well inside the 1e-4 parity bar. The fusions are written out, not
// left to the compiler's contraction, so every kernel of this file that composes these terms rounds them the same
// way whatever the surrounding code and register schedule. The traversal arithmetic (walk distances, exit planes)
// is never fused, so the visited cells stay bit-exact.

__device__ __forceinline__ void blend_add(Blend& B, float m, float r, float g, float b) {
    if (m < B.m) {
        const float s = fexp(-0.5f * (B.m - m));
        B.a *= s, B.r *= s, B.g *= s, B.b *= s, B.m = m;
    }
    const float w = fexp(-0.5f * (m - B.m));
    B.a += w, B.r = fmaf(w, r, B.r), B.g = fmaf(w, g, B.g), B.b = fmaf(w, b, B.b);
}

// (vx, vy, vz) A (vx, vy, vz)^T for the symmetric conic A = (p.x p.y p.z / . p.w q.x / . . q.y)
__device__ __forceinline__ float maha_f(const float4& p, const float4& q, float vx, float vy, float vz) {
    const float diag = fmaf(p.x * vx, vx, fmaf(p.w * vy, vy, q.y * vz * vz));
    const float cross = fmaf(p.y * vx, vy, fmaf(p.z * vx, vz, q.x * vy * vz));
    return fmaf(2.f, cross, diag);
}

// Sample point o + t d, used by the field terms only (the traversal never reads it).
__device__ __forceinline__ void sample_point(const float (&o)[3], const float (&d)[3], float t, float (&x)[3]) {
    x[0] = fmaf(t, d[0], o[0]), x[1] = fmaf(t, d[1], o[1]), x[2] = fmaf(t, d[2], o[2]);
}

__device__ __forceinline__ void offset_of(const float (&x)[3], const float4& p, float& v0, float& v1, float& v2,
                                          float& r2) {
    v0 = x[0] - p.x, v1 = x[1] - p.y, v2 = x[2] - p.z;
    r2 = fmaf(v0, v0, fmaf(v1, v1, v2 * v2));
}

// rho_k G_k(x) from the density record (q0 = xx xy xz yy, q1 = yz zz min(raw, 30) 0).
__device__ __forceinline__ float density_term(const float4& q0, const float4& q1, float v0, float v1, float v2) {
    return fexp(fmaf(-0.5f, maha_f(q0, q1, v0, v1, v2), q1.z));
}

__device__ __forceinline__ float weight_of(float m, float mmin) { return fexp(-0.5f * (m - mmin)); }

__device__ __forceinline__ void accumulate(float& A, float& r, float& g, float& bl, float w, const float (&c)[3]) {
    A += w, r = fmaf(w, c[0], r), g = fmaf(w, c[1], g), bl = fmaf(w, c[2], bl);
}

// Adds blocks q0 .. q0 + 3 (those below nv) of a site's SH coefficients (fp32, or fp16 pairs) to c: the colour
// SH_k(d) accumulates over the coefficients in storage order, coefficient i of channel i mod 3 times basis i / 3.
template <bool HALF, int CH = 4>
__device__ __forceinline__ void sh_accumulate(const float4 (&f)[CH], int q0, int nv, const float (&b)[16],
                                              float (&c)[3]) {
#pragma unroll
    for (int uq = 0; uq < CH; ++uq) {
        const int q = q0 + uq;
        if (q >= nv) break;
        const float fv[4] = {f[uq].x, f[uq].y, f[uq].z, f[uq].w};
        if (HALF) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float2 p = cutoffs(fv[u]);
                const int i0 = 8 * q + 2 * u, i1 = i0 + 1;
                c[i0 % 3] = fmaf(b[i0 / 3], p.x, c[i0 % 3]);
                c[i1 % 3] = fmaf(b[i1 / 3], p.y, c[i1 % 3]);
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) c[(4 * q + u) % 3] = fmaf(b[(4 * q + u) / 3], fv[u], c[(4 * q + u) % 3]);
        }
    }
}

// ------------------------------------------------------------------ traversal arithmetic (never contracted)

// Colour blocks of site k for this ray come through the wave-shared LDS cache of SH coefficient blocks: SLOTS
// direct-mapped slots (site k mod SLOTS) plus `overflow` blocks used within one lookup, stored [12][blocks] float4
// so that lanes reading different slots hit different banks. The 64 rays of a tile read overlapping sets of sites
// (45 % of the lookups find their block in LDS on the config-3 scene); the colour itself, max(SH_k(d) + 1/2, 0), is
// evaluated per lane since it depends on the ray direction.
//
// n_sh (stats[:, 4]) is the reference's count: the colour lookups that miss its per-ray cache of 8 direct-mapped
// slots keyed by k & 7, each holding the last site looked up in it (foam_infer.cu:151-168). A hit there returns the
// colour computed at the earlier lookup, the same bits the SH evaluation gives, so only the tags are kept, in one of
// two ways:
// - with a slot table (TABLE; the colour cut-off is +inf, so a pass looks up every entry of the cell's
//   neighbourhood in CSR order): within one pass the sites are distinct, so a lookup can hit only as the first
//   entry of its slot in the pass, and only if the ray's tag of that slot is that site; after the pass the slot
//   holds its last entry. The table gives each site's first and last entry of every slot, so the 8 tags live in
//   registers and are checked and replaced once per pass, with static slot indices;
// - otherwise 8 tags per ray in the wave's LDS, checked and replaced at every lookup in the reference's order.
//
// Tuning per colour mode, measured on config 3. Fused and baked colours: 24 slots and 4 overflow blocks (5.8 KB of
// LDS per wave), so that 24 waves (6 per SIMD) fit in a CU's 160 KB, and no software pipelining: the registers that
// pipelined loads hold are worth more as a sixth wave, whose loads cover the latency instead (48 slots at 4 waves,
// 36 at 5 and 26 at 7 were all slower: 233, 216 and 257 ms against 207 without overflow blocks). Lazy colours take
// 36 slots and no overflow blocks at 5 waves and the pipelined loops (edge records two edges ahead, site records one
// ahead).
template <int COLOR>
struct Tune {
    static constexpr int slots = COLOR == kLazy ? 36 : 24;
    static constexpr int overflow = COLOR == kLazy ? 0 : 4;
    static constexpr int waves = COLOR == kLazy ? 5 : 6;
    static constexpr bool pipelined = COLOR == kLazy;
};

template <int SLOTS>
__device__ __forceinline__ int slot_of(int k) {
    return static_cast<int>(static_cast<uint32_t>(k) % SLOTS);
}

// Entry e of a neighbourhood [e0, e1) for a load issued ahead of the loop that may not run: clamped into the cell,
// and for an empty cell (no self entry, which no pack_foam pack has) to the entry before it, so the load stays in
// bounds whatever the offsets.
__device__ __forceinline__ int entry_in(int e, int e1) { return max(min(e, e1 - 1), 0); }

// Volatile ints typed as LDS: the election and tag accesses stay ds_read / ds_write. Through a generic pointer
// they would be flat accesses, after each of which the wave waits for all of its outstanding global loads.
typedef __attribute__((address_space(3))) volatile int lds_int;

// The cache of one wave for colour mode COLOR (Tune<COLOR>: `slots` cached slots and `overflow` blocks), and the
// reference's per-ray colour-cache tags of the wave's rays.
template <int COLOR>
struct ColorCache {
    float4* data;    // [12][slots + overflow] coefficient blocks: the cached slots, then the overflow blocks
    lds_int* tag;    // site held by each slot (-1: empty)
    lds_int* claim;  // election word of each slot
    lds_int* ovf_k;  // per slot, in the current lookup: the site its losers' leader fetches into an overflow block
    lds_int* ovf_b;  // ... and that block (-1: none)
    lds_int* req_k;  // sites fetched by the current fill ...
    lds_int* req_b;  // ... and their blocks
    lds_int* rtag;   // this ray's tag of slot 0 of the reference's per-ray cache; slot s at rtag[s * rays]
    int rays;        // rays per wave (the tags are stored [8][rays], conflict-free across the wave's rays)
};

constexpr int kRayTagSlots = 8;  // the reference's per-ray colour cache: 8 direct-mapped slots (k & 7)

// LDS footprint of the colour cache of a wave rendering RAYS rays, in float4 units (the words follow the coefficient
// blocks, then the per-ray tags).
template <int COLOR, int RAYS, bool TABLE>
constexpr int cache_vec4(bool sh) {
    constexpr int S = Tune<COLOR>::slots, O = Tune<COLOR>::overflow, TAGS = TABLE ? 0 : kRayTagSlots * RAYS;
    return sh ? 12 * (S + O) + (2 * S + (O > 0 ? 2 * S : 0) + 2 * (S + O) + TAGS + 3) / 4 : 1;
}

// Waves per SIMD a kernel is compiled for: Tune's count, or fewer when its LDS (the colour cache and, without the
// slot table, the per-ray tags) does not fit that many workgroups of one wave in a CU's 160 KB.
template <int COLOR, int RAYS, bool TABLE>
constexpr int waves_for(bool sh) {
    constexpr int kCuLds = 160 * 1024, kSimds = 4;
    const int fit = kCuLds / (16 * cache_vec4<COLOR, RAYS, TABLE>(sh)) / kSimds;
    return fit < Tune<COLOR>::waves ? (fit < 1 ? 1 : fit) : Tune<COLOR>::waves;
}

// Sets up the wave's cache; `ray` is the lane's ray within the wave (0 .. RAYS - 1). TABLE: no LDS tags.
template <int COLOR, int RAYS, bool TABLE>
__device__ __forceinline__ ColorCache<COLOR> make_cache(float4* lds, int ray) {
    constexpr int S = Tune<COLOR>::slots, O = Tune<COLOR>::overflow;
    ColorCache<COLOR> C;
    C.data = lds;
    C.tag = (lds_int*)(lds + 12 * (S + O));
    C.claim = C.tag + S;
    C.ovf_k = C.claim + S;
    C.ovf_b = C.ovf_k + (O > 0 ? S : 0);
    C.req_k = C.ovf_b + (O > 0 ? S : 0);
    C.req_b = C.req_k + S + O;
    C.rays = RAYS;
    C.rtag = C.req_b + S + O + ray;
    for (int i = threadIdx.x; i < S; i += kBlock) C.tag[i] = -1, C.claim[i] = -1;
    if (!TABLE)
        for (int i = threadIdx.x; i < kRayTagSlots * RAYS; i += kBlock) C.req_b[S + O + i] = -1;
    __syncthreads();
    return C;
}

// 1 if site k misses this ray's slot k & 7 of the reference's colour cache, which then holds k; a lane alone on its
// ray (one ray per lane).
template <int COLOR>
__device__ __forceinline__ int ray_tag_miss(ColorCache<COLOR>& C, int k) {
    lds_int* p = C.rtag + (k & (kRayTagSlots - 1)) * C.rays;
    const int held = *p;
    *p = k;
    return held != k ? 1 : 0;
}

// The same for a group of G lanes per ray whose lane g looks up site k when `look` is set, in one round of a
// neighbourhood pass: the reference's order of these lookups is lane 0, 1, ..., G - 1 (lane g takes the edges
// g, g + G, ... of the cell), so the lanes check and replace their tags in G steps of that order, one lane of every
// group per step. Called with the group's lanes converged (each lane's `look` says whether it looks up).
template <int G, int COLOR>
__device__ __forceinline__ int group_tag_miss(ColorCache<COLOR>& C, int g, bool look, int k) {
    lds_int* p = C.rtag + (k & (kRayTagSlots - 1)) * C.rays;
    int held = k;
#pragma unroll
    for (int j = 0; j < G; ++j) {
        if (look && g == j) held = *p, *p = k;
    }
    return held != k ? 1 : 0;
}

// Number of set bits of `mask` below this lane.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
    return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u)));
}

// max(SH_k(d) + 1/2, 0) for every active lane (the lanes that need a colour now; control flow is uniform across
// them), site k's coefficient block read through the wave cache.
//
// The SH basis of the ray's direction that a colour evaluation multiplies: held in registers for the whole ray, or,
// with 8 lanes per ray (memory-bound batches), evaluated at each lookup from the direction, which takes 16 registers
// out of the sample loop. The empty asm keeps the compiler from hoisting that evaluation out of the loops. Measured
// on config 5's 8-lane batch: 2271 -> 2207 ms (24 -> 12 spilled VGPRs), and 2171 ms (5, none stored in the sample
// loop) with the block read two float4 at a time in that evaluation. The one-ray-per-lane kernels keep the basis and
// four float4 at a time: two gave 20 spilled VGPRs instead of 24 there but 183.0 against 179.6 ms on config 3.
constexpr int kLateBasisLanes = 8;  // lanes per ray of the layout that evaluates the basis per lookup

// This lane's index in its wave, read from the hardware where it is needed (mbcnt over a full mask). Inside an asm
// statement the compiler cannot keep it in a register across loops, nor spill and reload it there.
__device__ __forceinline__ int lane_fresh() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

template <int DEG>
struct LateBasis {
    float x, y, z;
};

__device__ __forceinline__ void basis_fill(const float (&b)[16], float (&out)[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) out[i] = b[i];
}

template <int DEG>
__device__ __forceinline__ void basis_fill(const LateBasis<DEG>& L, float (&out)[16]) {
    float x = L.x, y = L.y, z = L.z;
    asm volatile("" : "+v"(x), "+v"(y), "+v"(z));
    sh_basis(x, y, z, DEG, out);
}

// The texture path and LDS charge a wave-wide load the same cycles however few of its lanes are active, and the
// evaluation (12 LDS reads, 48 FMAs) costs the wave the same however few of its lanes take part, so a lookup aims
// to serve every lane in one pass. Each pass:
// - lanes whose site is in its home slot (k mod SLOTS) pin it; the missing sites claim their home slots, the last
//   claim wins and tags the slot at once (the cache belongs to this wave, which reads a block only after the fill),
//   and lanes of the winner's site join it;
// - lanes whose home slot is pinned by, or went to, another site elect one leader per slot; the first `overflow`
//   leaders' sites get overflow blocks, which serve their lanes in this pass and are not cached;
// - all active lanes fetch the claimed blocks together (one float4 per lane per load), then every served lane reads
//   its block, four float4 at a time, multiplying as it goes.
// Lanes left over (more conflicts than overflow blocks, or a second site in one slot's losers) take another pass;
// every pass serves at least one lane, so the loop ends (after the first pass in about 4 lookups of 5 on config 3).
// Wave barriers separate the phases: the lanes of a phase act on what every lane did in the phase before, and the
// barrier is convergent, so the compiler cannot merge one-sided stores across it.
template <bool HALF, int NV, int COLOR, class BASIS>
__device__ __forceinline__ void cached_colour(ColorCache<COLOR>& C, const float4* __restrict__ sh, int stride, int k,
                                              const BASIS& basis, float (&c)[3]) {
    constexpr int SLOTS = Tune<COLOR>::slots, OVF = Tune<COLOR>::overflow, BLOCKS = SLOTS + OVF;
    const int lane = static_cast<int>(threadIdx.x);
    const int home = slot_of<SLOTS>(k);
    const uint64_t active = __ballot(1);
    const int n_active = __popcll(active), rank = lanes_below(active);
    bool pending = true;
    for (;;) {
        const bool hit = pending && C.tag[home] == k;
        const bool miss = pending && !hit;
        if (miss) C.claim[home] = lane;
        __builtin_amdgcn_wave_barrier();
        if (hit) C.claim[home] = -1;  // pin, after the claims
        __builtin_amdgcn_wave_barrier();
        const bool win = miss && C.claim[home] == lane;
        if (win) C.tag[home] = k;
        __builtin_amdgcn_wave_barrier();
        const bool lose = miss && !win && C.tag[home] != k;  // the slot holds another site in this lookup
        int block = home;
        bool served = hit || (miss && !lose), lead_fetch = false;
        if (OVF > 0 && __ballot(lose) != 0) {
            if (lose) C.claim[home] = lane;
            __builtin_amdgcn_wave_barrier();
            const bool lead = lose && C.claim[home] == lane;
            const uint64_t leads = __ballot(lead);
            if (lead) {
                const int o = lanes_below(leads);
                lead_fetch = o < OVF;
                C.ovf_k[home] = k, C.ovf_b[home] = lead_fetch ? SLOTS + o : -1;
            }
            __builtin_amdgcn_wave_barrier();
            if (lose) {
                const int ok = C.ovf_k[home], ob = C.ovf_b[home];
                if (ok == k && ob >= 0) block = ob, served = true;
            }
        }
        const bool fetch = win || lead_fetch;
        const uint64_t fetches = __ballot(fetch);
        if (fetches != 0) {
            if (fetch) {
                const int r = lanes_below(fetches);
                C.req_k[r] = k, C.req_b[r] = block;
            }
            __builtin_amdgcn_wave_barrier();
            const int total = NV * __popcll(fetches);
            for (int base = 0; base < total; base += n_active) {
                const int j = base + rank;
                if (j < total) {
                    const int r = j / NV, q = j - r * NV;
                    const int kr = C.req_k[r];
                    C.data[q * BLOCKS + C.req_b[r]] = sh[stride * static_cast<int64_t>(kr) + q];
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
        if (served) {
            float b[16];
            basis_fill(basis, b);
            // with the basis evaluated here, two float4 of the block at a time (else four)
            constexpr int CH = std::is_same_v<BASIS, float[16]> ? 4 : 2;
            c[0] = c[1] = c[2] = 0.5f;
#pragma unroll
            for (int q0 = 0; q0 < NV; q0 += CH) {
                float4 f[CH];
#pragma unroll
                for (int u = 0; u < CH; ++u)
                    if (q0 + u < NV) f[u] = C.data[(q0 + u) * BLOCKS + block];
                sh_accumulate<HALF, CH>(f, q0, NV, b, c);
                __builtin_amdgcn_sched_barrier(0);  // one chunk of the block in registers at a time
            }
            c[0] = fmaxf(c[0], 0.f), c[1] = fmaxf(c[1], 0.f), c[2] = fmaxf(c[2], 0.f);
        }
        pending = pending && !served;
        __builtin_amdgcn_wave_barrier();
        if (__ballot(pending) == 0) break;
    }
}

// The ray's tags of the slots a lane keeps (all 8 with one ray per lane; g, g + G, ... in a group of G lanes), for
// the slot-table accounting.
// The tags live in registers (static slot indices). Measured on config 3 against keeping them in the lane's scratch
// memory (read and written once per pass: 192.3 ms), in LDS (which takes colour-cache blocks: 201.5 ms) or packed
// 20 bits per tag (181.2 ms): 180.0 ms, against 172.9 with no tag work.
template <int G>
struct SlotTags {
    static constexpr int n = kRayTagSlots / G;
    int t[n];
};

template <int G>
__device__ __forceinline__ void tags_init(SlotTags<G>& T) {
#pragma unroll
    for (int i = 0; i < SlotTags<G>::n; ++i) T.t[i] = -1;
}

// One pass over the neighbourhood of cell c looked up every entry: returns the lookups of the lane's slots that hit
// the ray's cache (their first entry in the pass is the site the tag holds) and replaces those tags with the slots'
// last entries. Slot table row of site c: (F0, L0, F1, L1), ..., (F6, L6, F7, L7), first and last entry of each
// slot, -2 for a slot without entries.
template <int G>
__device__ __forceinline__ int table_hits(const FoamScene& S, int c, int g, SlotTags<G>& T) {
    const int4* row = S.slots + 4 * static_cast<int64_t>(c);
    int hits = 0;
    if constexpr (G == 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // slots 2q and 2q + 1
            const int4 v = row[q];
            hits += v.x == T.t[2 * q] ? 1 : 0;
            T.t[2 * q] = v.y >= 0 ? v.y : T.t[2 * q];
            hits += v.z == T.t[2 * q + 1] ? 1 : 0;
            T.t[2 * q + 1] = v.w >= 0 ? v.w : T.t[2 * q + 1];
            __builtin_amdgcn_sched_barrier(0);  // one int4 of the row in registers at a time
        }
    } else {
        const int2* fl = reinterpret_cast<const int2*>(row);
#pragma unroll
        for (int i = 0; i < SlotTags<G>::n; ++i) {
            const int2 v = fl[g + G * i];
            hits += v.x == T.t[i] ? 1 : 0;
            T.t[i] = v.y >= 0 ? v.y : T.t[i];
        }
    }
    return hits;
}

// One ray per lane with fused colours (one pass per sample): the cells of the passes whose cache hits are still to
// be counted, and the ray's 8 tags, in the lane's private memory (the log is written at a varying index, so it and
// the tags stay out of registers); every kPassLog passes, and at the end of the ray, the logged passes are counted
// in order with the tags in registers for the while. Measured on config 3 against the tags in registers: 179.4 and
// 179.3 ms (16 and 32 passes) against 179.8, 24 spilled VGPRs against 44; 64 passes 208.9 ms; for exact colours,
// whose passes follow the samples' weights, 227.4 against 182.8 ms, so they keep the tags in registers.
constexpr int kPassLog = 16;
struct PassLog {
    int mem[kPassLog + kRayTagSlots];  // cells of the logged passes, then the tags
    int n;
};

__device__ __forceinline__ int log_flush(const FoamScene& S, PassLog& L) {
    SlotTags<1> T;
#pragma unroll
    for (int s = 0; s < kRayTagSlots; ++s) T.t[s] = L.mem[kPassLog + s];
    int hits = 0;
    for (int i = 0; i < L.n; ++i) hits += table_hits<1>(S, L.mem[i], 0, T);
#pragma unroll
    for (int s = 0; s < kRayTagSlots; ++s) L.mem[kPassLog + s] = T.t[s];
    L.n = 0;
    return hits;
}

// The slot-table count of one ray per lane, with the tags behind a pass log (above) or in registers: set-up, a pass
// over cell c that looked up every entry (returns the hits counted now: all of the log's when it fills up), and the
// end of the ray (the hits not counted yet).
__device__ __forceinline__ void tags_init(PassLog& L) {
    L.n = 0;
#pragma unroll
    for (int s = 0; s < kRayTagSlots; ++s) L.mem[kPassLog + s] = -1;
}
__device__ __forceinline__ int tags_pass(const FoamScene& S, PassLog& L, int c) {
    L.mem[L.n] = c;
    return ++L.n == kPassLog ? log_flush(S, L) : 0;
}
__device__ __forceinline__ int tags_finish(const FoamScene& S, PassLog& L) { return log_flush(S, L); }
__device__ __forceinline__ int tags_pass(const FoamScene& S, SlotTags<1>& T, int c) { return table_hits<1>(S, c, 0, T); }
__device__ __forceinline__ int tags_finish(const FoamScene&, SlotTags<1>&) { return 0; }

// Number of float4 a colour fetch reads: the blocks holding coefficients of degree <= DEG (the others multiply a
// zero basis value, so leaving them out changes no finite colour).
template <bool HALF, int DEG>
constexpr int sh_vec4() {
    return HALF ? sh_vec4_f16(DEG) : sh_vec4_f32(DEG);
}

// Greedy walk to the lexicographic argmin of (|x - p|^2, tie order) over {c} U adj(c), repeated. IDX: the edge
// records carry the neighbour index (indexed pack).
template <bool IDX = false>
__device__ int walk_to(const FoamScene& S, int c, float x0, float x1, float x2, int& steps) {
    for (int it = 0; it < kWalkCap; ++it) {
        const float4 pc = S.points[c];
        float bd = (x0 - pc.x) * (x0 - pc.x) + (x1 - pc.y) * (x1 - pc.y) + (x2 - pc.z) * (x2 - pc.z);
        int bk = c;
        const int e0 = S.offsets[c], e1 = S.offsets[c + 1];
        for (int e = e0 + 1; e < e1; ++e) {
            const float4 ed = S.edge[e];
            const int k = IDX ? __float_as_int(ed.w) : S.nbr[e];
            const float v0 = x0 - ed.x, v1 = x1 - ed.y, v2 = x2 - ed.z;
            const float dk = v0 * v0 + v1 * v1 + v2 * v2;
            if (dk < bd || (dk == bd && before(S, k, bk))) bd = dk, bk = k;
        }
        if (bk == c) break;
        c = bk;
        ++steps;
    }
    return c;
}

// Result of one pass over a cell's neighbourhood for one sample.
struct CellEval {
    float sigma, mmin, t_exit;
    int next;
    Blend B;
};

// Exit-face candidate of edge (c -> k): bisector-plane parameter ahead of the ray, reference arithmetic.
__device__ __forceinline__ void exit_candidate(const FoamScene& S, const float4& pc, const float4& ed, int k,
                                               const float (&o)[3], const float (&d)[3], CellEval& R) {
    const float n0 = ed.x - pc.x, n1 = ed.y - pc.y, n2 = ed.z - pc.z;
    const float dn = n0 * d[0] + n1 * d[1] + n2 * d[2];
    if (dn > 0.f) {
        const float m0 = 0.5f * (ed.x + pc.x) - o[0], m1 = 0.5f * (ed.y + pc.y) - o[1],
                    m2 = 0.5f * (ed.z + pc.z) - o[2];
        const float tt = (m0 * n0 + m1 * n1 + m2 * n2) / dn;
        if (tt < R.t_exit || (tt == R.t_exit && (R.next == INT_MAX || before(S, k, R.next)))) R.t_exit = tt, R.next = k;
    }
}

// Site records of neighbour k read by a pass: density (q0, q1) from stage 1, colour conic (q2, q3) from stage 2.
struct SiteRec {
    float4 q0, q1, q2, q3;
};

// The group layout's site records: the site rows when the caller gives them, else the attr rows. The rows are 64
// bytes apart (one 128-byte line holds two whole rows, where 3 of 8 of the 80-byte attr rows straddle two lines), or
// 256 bytes apart in site blocks whose last 192 bytes hold the site's fp32 SH row: the record and the SH row of a
// neighbour visit then take two 128-byte lines, where a row and a separate 192-byte SH row take three.
__device__ __forceinline__ const float4* group_row(const FoamScene& S, int k) {
    return S.rows != nullptr ? S.rows + S.row_stride * static_cast<int64_t>(k) : S.attr + 5 * static_cast<int64_t>(k);
}

template <int STAGE>
__device__ __forceinline__ SiteRec group_site_rec(const FoamScene& S, int k) {
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    SiteRec r{zero4, zero4, zero4, zero4};
    const float4* a = group_row(S, k);
    if (STAGE >= 1) r.q0 = a[0], r.q1 = a[1];
    if (STAGE >= 2) r.q2 = a[2], r.q3 = a[3];
    return r;
}

template <int STAGE>
__device__ __forceinline__ SiteRec site_rec(const FoamScene& S, int k) {
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    SiteRec r{zero4, zero4, zero4, zero4};
    const float4* a = S.attr + 5 * static_cast<int64_t>(k);
    if (STAGE >= 1) r.q0 = a[0], r.q1 = a[1];
    if (STAGE >= 2) r.q2 = a[2], r.q3 = a[3];
    return r;
}

// One pass over the self-first neighbourhood of cell c for the sample o + t d: density, smallest colour
// Mahalanobis distance (lazy) or running colour blend (fused, baked), and, when want_exit, the exit face.
// Pipelined (Tune): the edge record of e + 2 and the site records of e + 1 are loaded while edge e is evaluated,
// indices clamped to the cell so every load stays in bounds.
template <int STAGE, int COLOR, bool HALF, int DEG, bool TABLE>
__device__ void eval_cell(const FoamScene& S, const FoamParams& P, int c, float t, const float (&o)[3],
                          const float (&d)[3], const float (&b)[16], ColorCache<COLOR>& cache,
                          bool want_exit, CellEval& R, int& n_dens, int& n_sh) {
    constexpr bool BLEND = STAGE >= 2 && COLOR != kLazy;
    // Fused blend: the edge record of e + 1 (and, on the reference records, its neighbour index) is requested in
    // round e, after the density term and before the colour lookup, whose latency then covers it; round e + 1
    // starts with its neighbour index in hand. (Issued at the top of the round it spills the loop's registers; at
    // its end it arrives too late to help. Baked colours, with no lookup to cover it, run slower with it.) The
    // first record requested is the cell's own (self-first), which holds its position: on the reference records
    // the cell position is taken from it (fewer spilled VGPRs there; on the indexed records the separate load is
    // faster).
    constexpr bool IDX = COLOR == kFusedIdx, PREF = STAGE >= 2 && (COLOR == kFused || IDX);
    const int e0 = S.offsets[c], e1 = S.offsets[c + 1];
    const int last = e1 - 1;
    float4 edn;
    int kn = 0;
    if constexpr (PREF) {
        edn = S.edge[entry_in(e0, e1)];
        if constexpr (!IDX) kn = S.nbr[entry_in(e0, e1)];
    }
    const float4 pc = PREF && !IDX ? edn : S.points[c];
    float x[3];
    sample_point(o, d, t, x);
    R.sigma = 0.f, R.mmin = kInf, R.t_exit = kInf, R.next = INT_MAX;
    blend_init(R.B);
    constexpr bool PIPE = Tune<COLOR>::pipelined;
    // the edge and site records of e (and, pipelined, of e + 1 and e + 2)
    float4 ed, ed1;
    int k, k1;
    SiteRec q;
    if constexpr (PIPE) {
        ed = S.edge[entry_in(e0, e1)], ed1 = S.edge[entry_in(e0 + 1, e1)];
        k = S.nbr[entry_in(e0, e1)], k1 = S.nbr[entry_in(e0 + 1, e1)];
        q = site_rec<STAGE>(S, k);
    }
    for (int e = e0; e < e1; ++e) {
        float4 ed2;
        int k2;
        SiteRec qn;
        if constexpr (PIPE) {
            const int e2 = min(e + 2, last);
            ed2 = S.edge[e2], k2 = S.nbr[e2];
            qn = site_rec<STAGE>(S, k1);
        } else if constexpr (PREF) {
            ed = edn, k = IDX ? __float_as_int(ed.w) : kn;
            q = site_rec<STAGE>(S, k);
        } else {
            ed = S.edge[e], k = S.nbr[e];
            q = site_rec<STAGE>(S, k);
        }
        if (want_exit && e > e0) exit_candidate(S, pc, ed, k, o, d, R);
        if (STAGE >= 1) {
            float v0, v1, v2, r2;
            offset_of(x, ed, v0, v1, v2, r2);
            const float2 cut = cutoffs(COLOR == kFusedIdx ? q.q1.w : ed.w);
            if (r2 <= cut.x) {
                R.sigma += density_term(q.q0, q.q1, v0, v1, v2);
                ++n_dens;
            }
            if constexpr (PREF) {
                const int en = min(e + 1, last);
                edn = S.edge[en];
                if constexpr (!IDX) kn = S.nbr[en];
            }
            if (STAGE >= 2) {
                const float lb = r2 * cut.y;
                if (BLEND) {
                    const float lim = R.B.m + P.color_cut;
                    if (lb <= lim) {
                        const float m = maha_f(q.q2, q.q3, v0, v1, v2);
                        if (m <= lim) {
                            float c3[3];
                            if (COLOR == kBaked) {
                                const float4 q4 = S.attr[5 * static_cast<int64_t>(k) + 4];
                                c3[0] = q4.x, c3[1] = q4.y, c3[2] = q4.z;
                            } else {
                                if constexpr (TABLE) ++n_sh;  // the pass's hits come off in table_hits
                                else n_sh += ray_tag_miss(cache, k);
                                cached_colour<HALF, sh_vec4<HALF, DEG>()>(cache, S.sh, HALF ? 6 : 12, k, b, c3);
                            }
                            blend_add(R.B, m, c3[0], c3[1], c3[2]);
                        }
                    }
                } else if (lb < R.mmin) {
                    R.mmin = fminf(R.mmin, maha_f(q.q2, q.q3, v0, v1, v2));
                }
            }
        }
        if constexpr (PIPE) ed = ed1, k = k1, ed1 = ed2, k1 = k2, q = qn;
    }
}

// Lazy colour of the sample o + t d in cell c, given its smallest colour Mahalanobis distance mmin (lazy mode only,
// pipelined as eval_cell is).
template <bool HALF, int DEG, bool TABLE>
__device__ void color_lazy(const FoamScene& S, const FoamParams& P, int c, float t, float mmin, const float (&o)[3],
                           const float (&d)[3], const float (&b)[16], ColorCache<kLazy>& cache,
                           float (&C)[3], int& n_sh) {
    float x[3];
    sample_point(o, d, t, x);
    const int e0 = S.offsets[c], e1 = S.offsets[c + 1];
    const int last = e1 - 1;
    const float cut = mmin + P.color_cut;
    float A = 0.f, r = 0.f, g = 0.f, bl = 0.f;
    constexpr bool PIPE = Tune<kLazy>::pipelined;
    float4 ed, ed1, q2, q3;
    int k, k1;
    if constexpr (PIPE) {
        ed = S.edge[entry_in(e0, e1)], ed1 = S.edge[entry_in(e0 + 1, e1)];
        k = S.nbr[entry_in(e0, e1)], k1 = S.nbr[entry_in(e0 + 1, e1)];
        q2 = S.attr[5 * static_cast<int64_t>(k) + 2], q3 = S.attr[5 * static_cast<int64_t>(k) + 3];
    }
    for (int e = e0; e < e1; ++e) {
        float4 ed2, n2, n3;
        int k2;
        if constexpr (PIPE) {
            const int e2 = min(e + 2, last);
            ed2 = S.edge[e2], k2 = S.nbr[e2];
            const float4* a = S.attr + 5 * static_cast<int64_t>(k1);
            n2 = a[2], n3 = a[3];
        } else {
            ed = S.edge[e], k = S.nbr[e];
            const float4* a = S.attr + 5 * static_cast<int64_t>(k);
            q2 = a[2], q3 = a[3];
        }
        float v0, v1, v2, r2;
        offset_of(x, ed, v0, v1, v2, r2);
        if (r2 * cutoffs(ed.w).y <= cut) {
            const float m = maha_f(q2, q3, v0, v1, v2);
            if (m <= cut) {
                float c3[3];
                if constexpr (TABLE) ++n_sh;
                else n_sh += ray_tag_miss(cache, k);
                cached_colour<HALF, sh_vec4<HALF, DEG>()>(cache, S.sh, HALF ? 6 : 12, k, b, c3);
                accumulate(A, r, g, bl, weight_of(m, mmin), c3);
            }
        }
        if constexpr (PIPE) ed = ed1, k = k1, ed1 = ed2, k1 = k2, q2 = n2, q3 = n3;
    }
    const float inv = 1.f / A;
    C[0] = r * inv, C[1] = g * inv, C[2] = bl * inv;
}

template <bool TRACE>
__device__ __forceinline__ void trace_cell(const FoamScene& S, const FoamOut& O, int64_t r, int s, int c) {
    if (TRACE && s < O.trace_cap) O.trace[r * O.trace_cap + s] = S.orig != nullptr ? S.orig[c] : c;
}

// The register allocation is bounded for waves_for waves per SIMD (Tune<COLOR>::waves unless the LDS allows fewer).
// Six waves per SIMD is the fastest occupancy measured for the fused fp32 degree-3 kernel on config 3 although it
// spills: 80 VGPRs, the rest of the ray's state (accumulated colour and depth, the basis) stored to scratch once
// per sample, outside the neighbourhood loop; at 4 waves it needs no spills and ran 27 % slower, at 7 it spills
// inside the loop.
//
// EXACT (fused colour modes, colour cut-off +inf, slot table): the exact (lazy) colour mode run by the one-pass blend.
// The exact colour of a sample is sum_k exp(-(m_k - m_min) / 2) c_k / sum_k exp(-(m_k - m_min) / 2) over every
// neighbour (the cut-off is +inf); the blend keeps the same two sums relative to the running minimum, rescaled as
// it falls, so the colours agree to rounding. The statistics are the exact mode's: a colour pass counts only where
// the exact mode runs one (segments with weight > w_thresh, for the segment's far sample and, when the segment
// before was not coloured, its near sample), with that pass's lookups (every entry, as the blend's pass looks up)
// and the ray's cache tags advanced by those passes alone.
template <int STAGE, int COLOR, bool HALF, int DEG, bool TRACE, bool TABLE, bool EXACT = false>
__global__ void __launch_bounds__(kBlock, (waves_for<COLOR, kBlock, TABLE>(STAGE >= 2 && COLOR != kBaked)))
    foam_infer_kernel(FoamScene S, FoamParams P, FoamRays R, FoamOut O) {
    static_assert(!EXACT || (TABLE && STAGE == 2 && (COLOR == kFused || COLOR == kFusedIdx)), "exact via the blend");
    constexpr bool kSH = STAGE >= 2 && COLOR != kBaked;
    constexpr bool BLEND = STAGE >= 2 && COLOR != kLazy;
    constexpr bool FUSED_SH = BLEND && COLOR != kBaked;
    __shared__ float4 cache_lds[cache_vec4<COLOR, kBlock, TABLE>(kSH)];
    ColorCache<COLOR> cache{};  // set up by every lane of the block before any returns
    if (kSH) cache = make_cache<COLOR, kBlock, TABLE>(cache_lds, static_cast<int>(threadIdx.x));
    const int64_t i = xcd_block_id() * kBlock + threadIdx.x;
    if (i >= R.n) return;
    const int64_t r = R.order != nullptr ? R.order[i] : i;
    if (r < 0 || r >= R.n) return;  // not a permutation entry: nothing is read or written
    const int start = R.start[r];
    if (start < 0 || start >= S.n_sites) {  // not traced: empty foreground
        O.rgb[3 * r] = O.rgb[3 * r + 1] = O.rgb[3 * r + 2] = 0.f;
        O.T[r] = 1.f, O.depth[r] = 0.f;
#pragma unroll
        for (int i = 0; i < 5; ++i) O.stats[5 * r + i] = 0;
        return;
    }
    const float o[3] = {R.o[3 * r], R.o[3 * r + 1], R.o[3 * r + 2]};
    const float d[3] = {R.d[3 * r], R.d[3 * r + 1], R.d[3 * r + 2]};
    const float t_near = R.t_near[r], t_far = R.t_far[r];
    const int max_samples = R.cap != nullptr ? R.cap[r] : INT_MAX;
    float b[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) b[i] = 0.f;
    if (kSH) sh_basis(d[0], d[1], d[2], DEG, b);

    int walk_steps = 0, n_dens = 0, n_sh = 0;
    std::conditional_t<TABLE && FUSED_SH && !EXACT, PassLog, SlotTags<1>> tags;
    tags_init(tags);
    int c = walk_to<COLOR == kFusedIdx>(S, start, o[0] + t_near * d[0], o[1] + t_near * d[1], o[2] + t_near * d[2],
                                        walk_steps);
    CellEval E;
    int looks = 0, looksP = 0;  // EXACT: lookups of the latest pass and of the one before
    bool litP = false;          // EXACT: the segment ending at the near sample was coloured
    eval_cell<STAGE, COLOR, HALF, DEG, TABLE>(S, P, c, t_near, o, d, b, cache, true, E, n_dens,
                                              EXACT ? looks : n_sh);
    if (TABLE && FUSED_SH && !EXACT) n_sh -= tags_pass(S, tags, c);
    trace_cell<TRACE>(S, O, r, 0, c);
    float sP = E.sigma, mP = E.mmin, tP = t_near, CP[3] = {0.f, 0.f, 0.f};
    bool hasP = false;
    int cP = c;
    if (BLEND) {
        const float inv = 1.f / E.B.a;
        CP[0] = E.B.r * inv, CP[1] = E.B.g * inv, CP[2] = E.B.b * inv, hasP = true;
    }
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f}, dep = 0.f;
    int n_samples = 1, n_color = 0;
    for (int it = 0; it < kMaxCells; ++it) {
        const bool last = E.next == INT_MAX || E.t_exit >= t_far || n_samples + 1 >= max_samples;
        const float tQ = last ? t_far : fmaxf(E.t_exit, tP);
        const int cQ = last ? c : E.next;
        looksP = looks, looks = 0;
        eval_cell<STAGE, COLOR, HALF, DEG, TABLE>(S, P, cQ, tQ, o, d, b, cache, !last, E, n_dens,
                                                  EXACT ? looks : n_sh);
        if (TABLE && FUSED_SH && !EXACT) n_sh -= tags_pass(S, tags, cQ);
        trace_cell<TRACE>(S, O, r, n_samples, cQ);
        ++n_samples;
        const float sQ = E.sigma, mQ = E.mmin;
        const float delta = tQ - tP;
        const float alpha = 1.f - fexp(-0.5f * (sP + sQ) * delta);
        const float w = T * alpha;
        float CQ[3] = {0.f, 0.f, 0.f};
        bool hasQ = false;
        if (BLEND) {
            const float inv = 1.f / E.B.a;
            CQ[0] = E.B.r * inv, CQ[1] = E.B.g * inv, CQ[2] = E.B.b * inv, hasQ = true;
        }
        const bool lit = STAGE >= 2 && w > P.w_thresh;
        if (lit) {
            if constexpr (EXACT) {
                if (!litP) n_sh += looksP - tags_pass(S, tags, cP);
                n_sh += looks - tags_pass(S, tags, cQ);
            }
            if constexpr (!BLEND) {
                if (!hasP) {
                    color_lazy<HALF, DEG, TABLE>(S, P, cP, tP, mP, o, d, b, cache, CP, n_sh);
                    if (TABLE) n_sh -= tags_pass(S, tags, cP);
                }
                color_lazy<HALF, DEG, TABLE>(S, P, cQ, tQ, mQ, o, d, b, cache, CQ, n_sh);
                if (TABLE) n_sh -= tags_pass(S, tags, cQ);
                hasQ = true;
            }
#pragma unroll
            for (int a = 0; a < 3; ++a) acc[a] += w * 0.5f * (CP[a] + CQ[a]);
            dep += w * 0.5f * (tP + tQ);
            ++n_color;
        }
        T *= 1.f - alpha;
        tP = tQ, sP = sQ, mP = mQ, hasP = hasQ, cP = cQ, c = cQ, litP = lit;
#pragma unroll
        for (int a = 0; a < 3; ++a) CP[a] = CQ[a];
        if (last || T < P.t_thresh) break;
    }
    if (TABLE && kSH) n_sh -= tags_finish(S, tags);
#pragma unroll
    for (int a = 0; a < 3; ++a) O.rgb[3 * r + a] = acc[a];
    O.T[r] = T;
    O.depth[r] = dep;
    int* st = O.stats + 5 * r;
    st[0] = n_samples, st[1] = n_color, st[2] = walk_steps, st[3] = n_dens, st[4] = n_sh;
}

// ------------------------------------------------------------------ group-per-ray layout
//
// The other wave64 layout: a group of G lanes (2, 4 or 8) serves one ray, 64 / G rays per wave (consecutive rays of
// the host's pixel tiles). Lane g of the group takes edges e0 + g, e0 + g + G, ... of each cell's self-first
// neighbourhood: its exit candidates, density terms and colour terms. The group then combines them with DPP row
// permutations (xor 1, then xor 2 within a quad, then the half-row mirror i <-> 7 - i): the exit face is the
// lexicographic minimum of (t, tie order), the same face as a sequential scan, so the visited cells are identical;
// sums (density, lazy colour weights, the sample statistics) and fused colour blends are combined in a butterfly,
// whose pairwise operations are commutative, so every lane of the group ends with the same bits and the group
// runs the compositing in lockstep. Only the summation order of the field terms differs from a sequential scan
// (a few ulps). Per lane this layout runs the same face and field arithmetic as one ray per lane, but 64 / G rays
// per wave keep more independent loads in flight per wave, and a wave's loads of one cell are contiguous.


__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// k precedes j in the tie order, INT_MAX (no face) after every site.
__device__ __noinline__ bool before_or_none(const FoamScene& S, int k, int j) {
    if (j == INT_MAX) return k != INT_MAX;
    if (k == INT_MAX) return false;
    return before(S, k, j);
}

// Keeps the lexicographic minimum of (t, k) and the candidate (u, j). Exact ties in t are rare: they take a
// wave-uniform branch, inside which only the tied lanes look up the tie order.
__device__ __forceinline__ void keep_min(const FoamScene& S, float u, int j, float& t, int& k) {
    bool take = u < t;
    const bool tie = u == t && j != k;
    if (wave_any(tie)) {
        if (tie) take = before_or_none(S, j, k);
    }
    if (take) t = u, k = j;
}

template <int CTRL>
__device__ __forceinline__ void min_step(const FoamScene& S, float& t, int& k) {
    const float u = row_perm<CTRL>(t);
    const int j = row_perm<CTRL>(k);
    keep_min(S, u, j, t, k);
}

template <int G>
__device__ __forceinline__ void group_min(const FoamScene& S, float& t, int& k) {
    static_assert(G == 2 || G == 4 || G == 8, "group width");
    min_step<kXor1>(S, t, k);
    if constexpr (G >= 4) min_step<kXor2>(S, t, k);
    if constexpr (G == 8) min_step<kHalfMirror>(S, t, k);
}

template <int G, typename V>
__device__ __forceinline__ V group_sum(V v) {
    v = v + row_perm<kXor1>(v);
    if constexpr (G >= 4) v = v + row_perm<kXor2>(v);
    if constexpr (G == 8) v = v + row_perm<kHalfMirror>(v);
    return v;
}

template <int G>
__device__ __forceinline__ float group_fmin(float v) {
    v = fminf(v, row_perm<kXor1>(v));
    if constexpr (G >= 4) v = fminf(v, row_perm<kXor2>(v));
    if constexpr (G == 8) v = fminf(v, row_perm<kHalfMirror>(v));
    return v;
}

// Two running blends combined: both rescaled to the smaller Mahalanobis distance. The products are rounded
// separately (no contraction), so merge(A, B) and merge(B, A) give the same bits.
template <int CTRL>
__device__ __forceinline__ void blend_step(Blend& B) {
    const float m2 = row_perm<CTRL>(B.m), a2 = row_perm<CTRL>(B.a), r2 = row_perm<CTRL>(B.r),
                g2 = row_perm<CTRL>(B.g), b2 = row_perm<CTRL>(B.b);
    const float m = fminf(B.m, m2);
    const float s1 = fexp(-0.5f * (B.m - m)), s2 = fexp(-0.5f * (m2 - m));
    const float pa = B.a * s1, qa = a2 * s2, pr = B.r * s1, qr = r2 * s2;
    const float pg = B.g * s1, qg = g2 * s2, pb = B.b * s1, qb = b2 * s2;
    B.a = pa + qa, B.r = pr + qr, B.g = pg + qg, B.b = pb + qb, B.m = m;
}

template <int G>
__device__ __forceinline__ void group_blend(Blend& B) {
    blend_step<kXor1>(B);
    if constexpr (G >= 4) blend_step<kXor2>(B);
    if constexpr (G == 8) blend_step<kHalfMirror>(B);
}

template <int G>
__device__ int walk_group(const FoamScene& S, int c, int g, float x0, float x1, float x2, int& steps) {
    for (int it = 0; it < kWalkCap; ++it) {
        const float4 pc = S.points[c];
        float bd = (x0 - pc.x) * (x0 - pc.x) + (x1 - pc.y) * (x1 - pc.y) + (x2 - pc.z) * (x2 - pc.z);
        int bk = c;
        const int e0 = S.offsets[c], e1 = S.offsets[c + 1];
        for (int e = e0 + 1 + g; e < e1; e += G) {
            const float4 ed = S.edge[e];
            const int k = S.nbr[e];
            const float v0 = x0 - ed.x, v1 = x1 - ed.y, v2 = x2 - ed.z;
            keep_min(S, v0 * v0 + v1 * v1 + v2 * v2, k, bd, bk);
        }
        group_min<G>(S, bd, bk);
        if (bk == c) break;
        c = bk;
        ++steps;
    }
    return c;
}

// eval_cell for lane g of a group: the lane's share of the neighbourhood, then the group reductions.
template <int STAGE, int COLOR, bool HALF, int DEG, int G, bool TABLE>
__device__ void eval_cell_group(const FoamScene& S, const FoamParams& P, int c, int g_in, float t,
                                const float (&o)[3], const float (&d)[3], const float (&b)[16],
                                ColorCache<COLOR>& cache, bool want_exit, CellEval& R, int& n_dens, int& n_sh) {
    constexpr bool BLEND = STAGE >= 2 && COLOR != kLazy;
    // the lane's place in its group (blocks of one wave): with 8 lanes per ray read afresh, not held across samples
    const int g = G == kLateBasisLanes ? lane_fresh() % G : g_in;
    const float4 pc = S.points[c];
    float x[3];
    sample_point(o, d, t, x);
    const int e0 = S.offsets[c], e1 = S.offsets[c + 1];
    R.sigma = 0.f, R.mmin = kInf, R.t_exit = kInf, R.next = INT_MAX;
    blend_init(R.B);
    // Fused blend: the lane's next edge record and neighbour index are requested mid-round, as in eval_cell
    // (indices clamped to the cell: a lane without a further edge reads the cell's last one).
    constexpr bool PREF = STAGE >= 2 && COLOR == kFused;
    float4 edn;
    int kn = 0;
    if constexpr (PREF) {
        const int ef = entry_in(e0 + g, e1);
        edn = S.edge[ef], kn = S.nbr[ef];
    }
    for (int e = e0 + g; e < e1; e += G) {
        const float4 ed = PREF ? edn : S.edge[e];
        const int k = PREF ? kn : S.nbr[e];
        const SiteRec q = group_site_rec<STAGE>(S, k);
        if (want_exit && e > e0) {
            const float n0 = ed.x - pc.x, n1 = ed.y - pc.y, n2 = ed.z - pc.z;
            const float dn = n0 * d[0] + n1 * d[1] + n2 * d[2];
            if (dn > 0.f) {
                const float m0 = 0.5f * (ed.x + pc.x) - o[0], m1 = 0.5f * (ed.y + pc.y) - o[1],
                            m2 = 0.5f * (ed.z + pc.z) - o[2];
                keep_min(S, (m0 * n0 + m1 * n1 + m2 * n2) / dn, k, R.t_exit, R.next);
            }
        }
        if (STAGE >= 1) {
            float v0, v1, v2, r2;
            offset_of(x, ed, v0, v1, v2, r2);
            const float2 cut = cutoffs(ed.w);
            if (r2 <= cut.x) {
                R.sigma += density_term(q.q0, q.q1, v0, v1, v2);
                ++n_dens;
            }
            if constexpr (PREF) {
                const int en = min(e + G, e1 - 1);
                edn = S.edge[en], kn = S.nbr[en];
            }
            if (STAGE >= 2) {
                const float lb = r2 * cut.y;
                if (BLEND) {
                    const float lim = R.B.m + P.color_cut;
                    float m = kInf;
                    if (lb <= lim) m = maha_f(q.q2, q.q3, v0, v1, v2);
                    const bool look = lb <= lim && m <= lim;
                    if (COLOR != kBaked) {
                        if constexpr (TABLE) n_sh += look ? 1 : 0;  // the pass's hits come off in table_hits
                        else n_sh += group_tag_miss<G>(cache, g, look, k);  // the group's lanes converged
                    }
                    if (look) {
                        float c3[3];
                        if (COLOR == kBaked) {
                            const float4 q4 = S.attr[5 * static_cast<int64_t>(k) + 4];
                            c3[0] = q4.x, c3[1] = q4.y, c3[2] = q4.z;
                        } else {
                            if constexpr (G == kLateBasisLanes)
                                cached_colour<HALF, sh_vec4<HALF, DEG>()>(cache, S.sh, S.sh_stride, k,
                                                                         LateBasis<DEG>{d[0], d[1], d[2]}, c3);
                            else
                                cached_colour<HALF, sh_vec4<HALF, DEG>()>(cache, S.sh, S.sh_stride, k, b, c3);
                        }
                        blend_add(R.B, m, c3[0], c3[1], c3[2]);
                    }
                } else if (lb < R.mmin) {
                    R.mmin = fminf(R.mmin, maha_f(q.q2, q.q3, v0, v1, v2));
                }
            }
        }
    }
    if (want_exit) group_min<G>(S, R.t_exit, R.next);
    if (STAGE >= 1) R.sigma = group_sum<G>(R.sigma);
    if (STAGE >= 2 && !BLEND) R.mmin = group_fmin<G>(R.mmin);
    if (BLEND) group_blend<G>(R.B);
}

// color_lazy for lane g of a group: weights relative to the group's mmin, so the colour-cut tests are those of a
// sequential scan; the weighted sums are combined at the end.
template <bool HALF, int DEG, int G, bool TABLE>
__device__ void color_lazy_group(const FoamScene& S, const FoamParams& P, int c, int g, float t, float mmin,
                                 const float (&o)[3], const float (&d)[3], const float (&b)[16],
                                 ColorCache<kLazy>& cache, float (&C)[3], int& n_sh) {
    float x[3];
    sample_point(o, d, t, x);
    const int e0 = S.offsets[c], e1 = S.offsets[c + 1];
    const float cut = mmin + P.color_cut;
    float A = 0.f, r = 0.f, gr = 0.f, bl = 0.f;
    for (int e = e0 + g; e < e1; e += G) {
        const float4 ed = S.edge[e];
        const int k = S.nbr[e];
        const float4* a = group_row(S, k);
        const float4 q2 = a[2], q3 = a[3];
        float v0, v1, v2, r2;
        offset_of(x, ed, v0, v1, v2, r2);
        const bool near_enough = r2 * cutoffs(ed.w).y <= cut;
        float m = kInf;
        if (near_enough) m = maha_f(q2, q3, v0, v1, v2);
        const bool look = near_enough && m <= cut;
        if constexpr (TABLE) n_sh += look ? 1 : 0;
        else n_sh += group_tag_miss<G>(cache, g, look, k);  // the group's lanes converged
        if (look) {
            float c3[3];
            if constexpr (G == kLateBasisLanes)
                cached_colour<HALF, sh_vec4<HALF, DEG>()>(cache, S.sh, S.sh_stride, k, LateBasis<DEG>{d[0], d[1], d[2]},
                                                         c3);
            else
                cached_colour<HALF, sh_vec4<HALF, DEG>()>(cache, S.sh, S.sh_stride, k, b, c3);
            accumulate(A, r, gr, bl, weight_of(m, mmin), c3);
        }
    }
    A = group_sum<G>(A), r = group_sum<G>(r), gr = group_sum<G>(gr), bl = group_sum<G>(bl);
    const float inv = 1.f / A;
    C[0] = r * inv, C[1] = gr * inv, C[2] = bl * inv;
}

// foam_infer_kernel with a group of G lanes per ray; same outputs (the group's lane 0 writes them).
template <int STAGE, int COLOR, bool HALF, int DEG, bool TRACE, int G, bool TABLE>
__global__ void __launch_bounds__(kBlock, (waves_for<COLOR, kBlock / G, TABLE>(STAGE >= 2 && COLOR != kBaked)))
    foam_group_kernel(FoamScene S, FoamParams P, FoamRays R, FoamOut O) {
    constexpr bool kSH = STAGE >= 2 && COLOR != kBaked;
    constexpr bool BLEND = STAGE >= 2 && COLOR != kLazy;
    constexpr bool FUSED_SH = BLEND && COLOR != kBaked;
    __shared__ float4 cache_lds[cache_vec4<COLOR, kBlock / G, TABLE>(kSH)];
    ColorCache<COLOR> cache{};  // set up by every lane of the block before any returns
    if (kSH) cache = make_cache<COLOR, kBlock / G, TABLE>(cache_lds, static_cast<int>(threadIdx.x) / G);
    const int g = static_cast<int>(threadIdx.x) % G;
    const int64_t i = xcd_block_id() * (kBlock / G) + threadIdx.x / G;
    if (i >= R.n) return;  // whole groups leave together
    int64_t r = R.order != nullptr ? R.order[i] : i;
    if (r < 0 || r >= R.n) return;
    const bool writer = g == 0;
    const int start = R.start[r];
    if (start < 0 || start >= S.n_sites) {  // not traced: empty foreground
        if (writer) {
            O.rgb[3 * r] = O.rgb[3 * r + 1] = O.rgb[3 * r + 2] = 0.f;
            O.T[r] = 1.f, O.depth[r] = 0.f;
#pragma unroll
            for (int i = 0; i < 5; ++i) O.stats[5 * r + i] = 0;
        }
        return;
    }
    const float o[3] = {R.o[3 * r], R.o[3 * r + 1], R.o[3 * r + 2]};
    const float d[3] = {R.d[3 * r], R.d[3 * r + 1], R.d[3 * r + 2]};
    const float t_near = R.t_near[r], t_far = R.t_far[r];
    const int max_samples = R.cap != nullptr ? R.cap[r] : INT_MAX;
    float b[16];  // unused with 8 lanes per ray, which evaluate it per lookup
#pragma unroll
    for (int i = 0; i < 16; ++i) b[i] = 0.f;
    if (kSH && G != kLateBasisLanes) sh_basis(d[0], d[1], d[2], DEG, b);

    int walk_steps = 0, n_dens = 0, n_sh = 0;
    SlotTags<G> tags;
    tags_init(tags);
    int c = walk_group<G>(S, start, g, o[0] + t_near * d[0], o[1] + t_near * d[1], o[2] + t_near * d[2], walk_steps);
    CellEval E;
    eval_cell_group<STAGE, COLOR, HALF, DEG, G, TABLE>(S, P, c, g, t_near, o, d, b, cache, true, E, n_dens, n_sh);
    if (TABLE && FUSED_SH) n_sh -= table_hits<G>(S, c, g, tags);
    if (writer) trace_cell<TRACE>(S, O, r, 0, c);
    float sP = E.sigma, mP = E.mmin, tP = t_near, CP[3] = {0.f, 0.f, 0.f};
    bool hasP = false;
    int cP = c;
    if (BLEND) {
        const float inv = 1.f / E.B.a;
        CP[0] = E.B.r * inv, CP[1] = E.B.g * inv, CP[2] = E.B.b * inv, hasP = true;
    }
    float T = 1.f, acc[3] = {0.f, 0.f, 0.f}, dep = 0.f;
    int n_samples = 1, n_color = 0;
    for (int it = 0; it < kMaxCells; ++it) {
        const bool last = E.next == INT_MAX || E.t_exit >= t_far || n_samples + 1 >= max_samples;
        const float tQ = last ? t_far : fmaxf(E.t_exit, tP);
        const int cQ = last ? c : E.next;
        eval_cell_group<STAGE, COLOR, HALF, DEG, G, TABLE>(S, P, cQ, g, tQ, o, d, b, cache, !last, E, n_dens, n_sh);
        if (TABLE && FUSED_SH) n_sh -= table_hits<G>(S, cQ, g, tags);
        if (writer) trace_cell<TRACE>(S, O, r, n_samples, cQ);
        ++n_samples;
        const float sQ = E.sigma, mQ = E.mmin;
        const float delta = tQ - tP;
        const float alpha = 1.f - fexp(-0.5f * (sP + sQ) * delta);
        const float w = T * alpha;
        float CQ[3] = {0.f, 0.f, 0.f};
        bool hasQ = false;
        if (BLEND) {
            const float inv = 1.f / E.B.a;
            CQ[0] = E.B.r * inv, CQ[1] = E.B.g * inv, CQ[2] = E.B.b * inv, hasQ = true;
        }
        if (STAGE >= 2 && w > P.w_thresh) {
            if constexpr (!BLEND) {
                if (!hasP) {
                    color_lazy_group<HALF, DEG, G, TABLE>(S, P, cP, g, tP, mP, o, d, b, cache, CP, n_sh);
                    if (TABLE) n_sh -= table_hits<G>(S, cP, g, tags);
                }
                color_lazy_group<HALF, DEG, G, TABLE>(S, P, cQ, g, tQ, mQ, o, d, b, cache, CQ, n_sh);
                if (TABLE) n_sh -= table_hits<G>(S, cQ, g, tags);
                hasQ = true;
            }
#pragma unroll
            for (int a = 0; a < 3; ++a) acc[a] += w * 0.5f * (CP[a] + CQ[a]);
            dep += w * 0.5f * (tP + tQ);
            ++n_color;
        }
        T *= 1.f - alpha;
        tP = tQ, sP = sQ, mP = mQ, hasP = hasQ, cP = cQ, c = cQ;
#pragma unroll
        for (int a = 0; a < 3; ++a) CP[a] = CQ[a];
        if (last || T < P.t_thresh) break;
    }
    n_dens = group_sum<G>(n_dens), n_sh = group_sum<G>(n_sh);
    if (G == kLateBasisLanes && !TRACE) {  // the ray index read again rather than held across the sample loop
        const int64_t i_end = xcd_block_id() * (kBlock / G) + lane_fresh() / G;
        r = R.order != nullptr ? R.order[i_end] : i_end;
    }
    if (writer) {
#pragma unroll
        for (int a = 0; a < 3; ++a) O.rgb[3 * r + a] = acc[a];
        O.T[r] = T;
        O.depth[r] = dep;
        int* st = O.stats + 5 * r;
        st[0] = n_samples, st[1] = n_color, st[2] = walk_steps, st[3] = n_dens, st[4] = n_sh;
    }
}

// Indexed edge records from a pack: edge_i[e] = (p_j, the bits of j = nbr[e]) for every entry, and attr_i = attr with
// column 7 (padding in the reference's layout) holding site k's cut-off word, which every edge record pointing at k
// carries in the reference's layout (the self entry's, edge[offsets[k]].w). One lane per float4 written.
__global__ void __launch_bounds__(256) index_pack_kernel(const int* __restrict__ offsets, const int* __restrict__ nbr,
                                                         const float4* __restrict__ edge, const float* __restrict__ attr,
                                                         int64_t n_sites, int64_t n_edges, float4* __restrict__ edge_i,
                                                         float* __restrict__ attr_i) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n_edges) {
        const float4 ed = edge[i];
        edge_i[i] = make_float4(ed.x, ed.y, ed.z, __int_as_float(nbr[i]));
        return;
    }
    const int64_t j = i - n_edges;  // one float of attr_i
    if (j >= 20 * n_sites) return;
    const int64_t k = j / 20;
    const int col = static_cast<int>(j - 20 * k);
    if (col != 7) {
        attr_i[j] = attr[j];
    } else {  // the self entry's word; 0 for a site without entries (never a neighbour of a consistent graph)
        const int e0 = offsets[k];
        attr_i[j] = e0 < offsets[k + 1] && e0 < n_edges ? edge[e0].w : 0.f;
    }
}

// The fused blend over the indexed edge records: one ray per lane (EXACT: the exact colour mode's statistics).
template <bool HALF, bool TRACE, bool TABLE, bool EXACT>
int launch_indexed(const FoamScene& S, const FoamParams& P, const FoamRays& R, const FoamOut& O, hipStream_t stream) {
    const dim3 grid(grid_for(R.n, kBlock)), block(kBlock);
    switch (P.sh_deg) {
        case 0: hipLaunchKernelGGL((foam_infer_kernel<2, kFusedIdx, HALF, 0, TRACE, TABLE, EXACT>), grid, block, 0, stream, S, P, R, O); break;
        case 1: hipLaunchKernelGGL((foam_infer_kernel<2, kFusedIdx, HALF, 1, TRACE, TABLE, EXACT>), grid, block, 0, stream, S, P, R, O); break;
        case 2: hipLaunchKernelGGL((foam_infer_kernel<2, kFusedIdx, HALF, 2, TRACE, TABLE, EXACT>), grid, block, 0, stream, S, P, R, O); break;
        default: hipLaunchKernelGGL((foam_infer_kernel<2, kFusedIdx, HALF, 3, TRACE, TABLE, EXACT>), grid, block, 0, stream, S, P, R, O);
    }
    return launch_status("foam_infer_kernel (indexed edges)");
}

// lanes: 1 = one ray per lane (foam_infer_kernel), 2, 4 or 8 = a group of that many lanes per ray
// (foam_group_kernel). TABLE: the reference's cache tags from the slot table (colour cut-off +inf).
template <int STAGE, int COLOR, bool HALF, int DEG, bool TRACE, bool TABLE = false>
int launch(const FoamScene& S, const FoamParams& P, const FoamRays& R, const FoamOut& O, int lanes,
           hipStream_t stream) {
    if (lanes == 2) {
        hipLaunchKernelGGL((foam_group_kernel<STAGE, COLOR, HALF, DEG, TRACE, 2, TABLE>),
                           dim3(grid_for(R.n, kBlock / 2)), dim3(kBlock), 0, stream, S, P, R, O);
        return launch_status("foam_group_kernel");
    }
    if (lanes == 4) {
        hipLaunchKernelGGL((foam_group_kernel<STAGE, COLOR, HALF, DEG, TRACE, 4, TABLE>),
                           dim3(grid_for(R.n, kBlock / 4)), dim3(kBlock), 0, stream, S, P, R, O);
        return launch_status("foam_group_kernel");
    }
    if (lanes == 8) {
        hipLaunchKernelGGL((foam_group_kernel<STAGE, COLOR, HALF, DEG, TRACE, 8, TABLE>),
                           dim3(grid_for(R.n, kBlock / 8)), dim3(kBlock), 0, stream, S, P, R, O);
        return launch_status("foam_group_kernel");
    }
    hipLaunchKernelGGL((foam_infer_kernel<STAGE, COLOR, HALF, DEG, TRACE, TABLE>), dim3(grid_for(R.n, kBlock)),
                       dim3(kBlock), 0, stream, S, P, R, O);
    return launch_status("foam_infer_kernel");
}

// Kernels with SH colours are specialised on the SH degree (block size and basis known at compile time) and on how
// they keep the reference's cache tags.
template <int COLOR, bool HALF, bool TRACE, bool TABLE>
int launch_deg(const FoamScene& S, const FoamParams& P, const FoamRays& R, const FoamOut& O, int lanes,
               hipStream_t stream) {
    switch (P.sh_deg) {
        case 0: return launch<2, COLOR, HALF, 0, TRACE, TABLE>(S, P, R, O, lanes, stream);
        case 1: return launch<2, COLOR, HALF, 1, TRACE, TABLE>(S, P, R, O, lanes, stream);
        case 2: return launch<2, COLOR, HALF, 2, TRACE, TABLE>(S, P, R, O, lanes, stream);
        default: return launch<2, COLOR, HALF, 3, TRACE, TABLE>(S, P, R, O, lanes, stream);
    }
}

template <int COLOR, bool HALF, bool TRACE>
int launch_sh(const FoamScene& S, const FoamParams& P, const FoamRays& R, const FoamOut& O, int lanes, bool table,
              hipStream_t stream) {
    return table ? launch_deg<COLOR, HALF, TRACE, true>(S, P, R, O, lanes, stream)
                 : launch_deg<COLOR, HALF, TRACE, false>(S, P, R, O, lanes, stream);
}

template <bool TRACE>
int dispatch(int stage, int color_mode, bool half, const FoamScene& S, const FoamParams& P, const FoamRays& R,
             const FoamOut& O, int lanes, bool table, hipStream_t stream) {
    if (stage == 0) return launch<0, kLazy, false, 0, TRACE>(S, P, R, O, lanes, stream);
    if (stage == 1) return launch<1, kLazy, false, 0, TRACE>(S, P, R, O, lanes, stream);
    if (color_mode == kBaked) return launch<2, kBaked, false, 0, TRACE>(S, P, R, O, lanes, stream);
    if (color_mode == kLazy)
        return half ? launch_sh<kLazy, true, TRACE>(S, P, R, O, lanes, table, stream)
                    : launch_sh<kLazy, false, TRACE>(S, P, R, O, lanes, table, stream);
    return half ? launch_sh<kFused, true, TRACE>(S, P, R, O, lanes, table, stream)
                : launch_sh<kFused, false, TRACE>(S, P, R, O, lanes, table, stream);
}

template <bool HALF>
int dispatch_indexed(bool trace, bool table, bool exact, const FoamScene& S, const FoamParams& P, const FoamRays& R,
                     const FoamOut& O, hipStream_t s) {
    if (exact)  // always with the slot table
        return trace ? launch_indexed<HALF, true, true, true>(S, P, R, O, s)
                     : launch_indexed<HALF, false, true, true>(S, P, R, O, s);
    if (trace)
        return table ? launch_indexed<HALF, true, true, false>(S, P, R, O, s)
                     : launch_indexed<HALF, true, false, false>(S, P, R, O, s);
    return table ? launch_indexed<HALF, false, true, false>(S, P, R, O, s)
                 : launch_indexed<HALF, false, false, false>(S, P, R, O, s);
}

// Slot table of the reference's per-ray colour cache: for site k, the first and the last entry of every slot
// (entry site j mod 8) of its self-first neighbourhood, in CSR order, -2 for a slot without entries; stored as
// (F0, L0, F1, L1), ..., (F6, L6, F7, L7). One lane per site.
__global__ void __launch_bounds__(256) slot_table_kernel(const int* __restrict__ offsets, const int* __restrict__ nbr,
                                                         int64_t n_sites, int4* __restrict__ slots) {
    const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k >= n_sites) return;
    int F[8], L[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) F[s] = L[s] = -2;
    const int e1 = offsets[k + 1];
    for (int e = offsets[k]; e < e1; ++e) {
        const int j = nbr[e];
        const int s = j & (kRayTagSlots - 1);
#pragma unroll
        for (int u = 0; u < 8; ++u) {  // static indices: the arrays stay in registers
            if (u == s) {
                F[u] = F[u] == -2 ? j : F[u];
                L[u] = j;
            }
        }
    }
    int4* row = slots + 4 * k;
#pragma unroll
    for (int q = 0; q < 4; ++q) row[q] = make_int4(F[2 * q], L[2 * q], F[2 * q + 1], L[2 * q + 1]);
}

// Lanes per ray of vgr_foam_infer and vgr_foam_infer_traced, the faster layout per path on config 3 (8.29M rays,
// 2M sites, SH degree 3). Traversal and density: 4 lanes per ray (stage 0: 42.6 ms against 60.6 with one ray per
// lane; stage 1: 59.3 against 67.2); lazy colours: 4 (262.8 against 276.6 ms). Fused and baked colours: one ray
// per lane (205.9 against 223.0, 249.9 and 290.6 ms at 2, 4 and 8 lanes; baked 107.6 against 109.3 at 2): their
// colour lookups run for every neighbour of every sample, and the 64 rays of a tile, in the same cell, step through
// its neighbours together, one site per lookup, where a group's lanes ask for different sites at once (29 % more
// VALU and LDS instructions per launch at 4 lanes).
constexpr int kDefaultLanes = 0;
inline int default_lanes(int64_t stage, int64_t color_mode) {
    return stage < 2 || color_mode == kLazy ? 4 : 1;
}

int foam_entry(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* nbr, const float* edge,
               int64_t n_edges, const float* attr, const void* sh, int32_t sh_half, int64_t sh_deg, const float* o,
               const float* d, const int32_t* start, const float* near_t, const float* far_t, int64_t n_rays,
               double t_thresh, double w_thresh, double color_cut, int64_t color_mode, int64_t stage,
               const int32_t* cap, const int32_t* orig, float* rgb, float* T, float* depth, int32_t* stats,
               int32_t* trace, int64_t trace_cap, const int32_t* order, int64_t lanes, void* stream,
               const float* edge_i = nullptr, const float* attr_i = nullptr, const int32_t* slots = nullptr,
               const float* rows = nullptr, int64_t row_floats = 16) {
    VGR_REQUIRE(n_rays >= 0, "foam_infer: n_rays must be >= 0 (got %lld)", static_cast<long long>(n_rays));
    // The indexed edge records serve the fused blend with one ray per lane (its default layout), and with the slot
    // table and the colour cut-off +inf the exact colours too, run by that blend (foam_infer_kernel, EXACT).
    const bool one_lane = lanes == kDefaultLanes || lanes == 1;
    const bool exact_blend = edge_i != nullptr && attr_i != nullptr && slots != nullptr && stage == 2 &&
                             color_mode == kLazy && one_lane && std::isinf(color_cut) && color_cut > 0;
    const bool indexed = exact_blend || (edge_i != nullptr && attr_i != nullptr && stage == 2 &&
                                         color_mode == kFused && one_lane);
    if (indexed) lanes = 1;
    if (lanes == kDefaultLanes) lanes = default_lanes(stage, color_mode);
    VGR_REQUIRE(lanes == 1 || lanes == 2 || lanes == 4 || lanes == 8,
                "foam_infer: lanes_per_ray must be 1, 2, 4 or 8 (got %lld)",
                static_cast<long long>(lanes));
    VGR_REQUIRE(color_mode >= kLazy && color_mode <= kFused,
                "color_mode must be 0 (lazy), 1 (baked) or 2 (fused)");
    VGR_REQUIRE(stage >= 0 && stage <= 2, "stage must be 0, 1 or 2");
    VGR_REQUIRE(sh_deg >= 0 && sh_deg <= 3, "sh_deg must be in [0, 3] (got %lld)", static_cast<long long>(sh_deg));
    if (n_rays == 0) return VGR_OK;
    VGR_REQUIRE(n_sites > 0 && n_sites <= INT_MAX, "foam_infer: n_sites must be in [1, 2^31) (got %lld)",
                static_cast<long long>(n_sites));
    VGR_REQUIRE(n_edges >= n_sites && n_edges <= INT_MAX, "foam_infer: n_edges must be in [N, 2^31) (got %lld)",
                static_cast<long long>(n_edges));
    VGR_REQUIRE(points && offsets && nbr && edge && attr, "foam_infer: null scene pointer");
    VGR_REQUIRE(o && d && start && near_t && far_t, "foam_infer: null ray pointer");
    VGR_REQUIRE(rgb && T && depth && stats, "foam_infer: null output pointer");
    const bool needs_sh = stage == 2 && color_mode != kBaked;
    VGR_REQUIRE(!needs_sh || sh != nullptr, "foam_infer: sh is required unless colors are baked");
    VGR_REQUIRE(row_floats == 16 || row_floats == 64, "foam_infer: row_floats must be 16 or 64 (got %lld)",
                static_cast<long long>(row_floats));
    VGR_REQUIRE(row_floats == 16 || rows == nullptr || sh_half == 0,
                "foam_infer: site blocks (row_floats 64) hold fp32 SH rows; sh_half must be 0");
    // Fused and baked blends with a finite colour cut skip a neighbour against the running minimum of the terms
    // before it in edge order; a lane of a group sees only its own share of them, so these run one ray per lane.
    if (stage == 2 && color_mode != kLazy && !(color_cut > 1e30)) lanes = 1;
    // The site rows serve the group layouts' fused blend (config 5's 8-lane batch: 2538.6 -> 2437.6 ms with the
    // 64-byte rows); the two-pass exact colours with 4 lanes per ray ran slower on them (268.9 against 258.3 ms on
    // config 3) and keep the attr rows, as the one-ray-per-lane kernels do. Site blocks also supply those kernels'
    // SH rows, 16 float4 apart after each 4-float4 record.
    const bool rows_used = rows != nullptr && !indexed && stage == 2 && color_mode == kFused && lanes > 1;
    const bool blocks = rows_used && row_floats == 64;
    const FoamScene S{reinterpret_cast<const float4*>(points),
                      offsets,
                      nbr,
                      reinterpret_cast<const float4*>(indexed ? edge_i : edge),
                      reinterpret_cast<const float4*>(indexed ? attr_i : attr),
                      !needs_sh ? nullptr
                      : blocks  ? reinterpret_cast<const float4*>(rows) + 4
                                : reinterpret_cast<const float4*>(sh),
                      orig,
                      reinterpret_cast<const int4*>(slots),
                      rows_used ? reinterpret_cast<const float4*>(rows) : nullptr,
                      static_cast<int>(n_sites),
                      static_cast<int>(row_floats / 4),
                      blocks ? 16 : sh_half != 0 ? 6 : 12};
    const FoamParams P{static_cast<float>(t_thresh), static_cast<float>(w_thresh), static_cast<float>(color_cut),
                       static_cast<int>(sh_deg)};
    const FoamRays R{o, d, start, near_t, far_t, cap, n_rays, order};
    const FoamOut O{rgb, T, depth, stats, trace, trace_cap};
    const hipStream_t s = as_stream(stream);
    // The slot table gives the reference's cache misses per pass when a pass looks up every entry: colour cut-off
    // +inf (a pass with a finite cut-off skips entries, and keeps its tags in LDS per lookup). With 8 lanes per ray
    // (incoherent batches, bound by DRAM) the table's reads cost more than the per-lookup tags, which need only
    // 256 bytes of LDS per wave there: config 5's batch ran 2437.6 ms with the table, 2298.0 ms with the tags.
    const bool table = slots != nullptr && std::isinf(color_cut) && color_cut > 0 && lanes != 8;
    if (indexed)
        return sh_half != 0 ? dispatch_indexed<true>(trace != nullptr, table, exact_blend, S, P, R, O, s)
                            : dispatch_indexed<false>(trace != nullptr, table, exact_blend, S, P, R, O, s);
    if (trace != nullptr)
        return dispatch<true>(int(stage), int(color_mode), sh_half != 0, S, P, R, O, int(lanes), table, s);
    return dispatch<false>(int(stage), int(color_mode), sh_half != 0, S, P, R, O, int(lanes), table, s);
}

}  // namespace
}  // namespace vgr

extern "C" int vgr_foam_infer(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* nbr,
                              const float* edge, int64_t n_edges, const float* attr, const void* sh, int32_t sh_half,
                              int64_t sh_deg, const float* o, const float* d, const int32_t* start,
                              const float* near_t, const float* far_t, int64_t n_rays, double t_thresh,
                              double w_thresh, double color_cut, int64_t color_mode, int64_t stage,
                              const int32_t* cap, const int32_t* orig, float* rgb, float* T, float* depth,
                              int32_t* stats, void* stream) {
    return vgr::foam_entry(points, n_sites, offsets, nbr, edge, n_edges, attr, sh, sh_half, sh_deg, o, d, start,
                           near_t, far_t, n_rays, t_thresh, w_thresh, color_cut, color_mode, stage, cap, orig, rgb,
                           T, depth, stats, nullptr, 0, nullptr, vgr::kDefaultLanes, stream);
}

extern "C" int vgr_foam_infer_traced(const float* points, int64_t n_sites, const int32_t* offsets,
                                     const int32_t* nbr, const float* edge, int64_t n_edges, const float* attr,
                                     const void* sh, int32_t sh_half, int64_t sh_deg, const float* o, const float* d,
                                     const int32_t* start, const float* near_t, const float* far_t, int64_t n_rays,
                                     double t_thresh, double w_thresh, double color_cut, int64_t color_mode,
                                     int64_t stage, const int32_t* cap, const int32_t* orig, float* rgb, float* T,
                                     float* depth, int32_t* stats, int32_t* trace, int64_t trace_cap,
                                     void* stream) {
    VGR_REQUIRE(trace != nullptr && trace_cap > 0, "foam_infer_traced: trace must be non-null with trace_cap > 0");
    return vgr::foam_entry(points, n_sites, offsets, nbr, edge, n_edges, attr, sh, sh_half, sh_deg, o, d, start,
                           near_t, far_t, n_rays, t_thresh, w_thresh, color_cut, color_mode, stage, cap, orig, rgb,
                           T, depth, stats, trace, trace_cap, nullptr, vgr::kDefaultLanes, stream);
}

extern "C" int vgr_foam_infer_lanes(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* nbr,
                                    const float* edge, int64_t n_edges, const float* attr, const void* sh,
                                    int32_t sh_half, int64_t sh_deg, const float* o, const float* d,
                                    const int32_t* start, const float* near_t, const float* far_t, int64_t n_rays,
                                    double t_thresh, double w_thresh, double color_cut, int64_t color_mode,
                                    int64_t stage, const int32_t* cap, const int32_t* orig, float* rgb, float* T,
                                    float* depth, int32_t* stats, int32_t* trace, int64_t trace_cap,
                                    const int32_t* order, int64_t lanes_per_ray, const int32_t* slots,
                                    void* stream) {
    VGR_REQUIRE(trace == nullptr || trace_cap > 0, "foam_infer_lanes: trace needs trace_cap > 0");
    return vgr::foam_entry(points, n_sites, offsets, nbr, edge, n_edges, attr, sh, sh_half, sh_deg, o, d, start,
                           near_t, far_t, n_rays, t_thresh, w_thresh, color_cut, color_mode, stage, cap, orig, rgb,
                           T, depth, stats, trace, trace == nullptr ? 0 : trace_cap, order, lanes_per_ray, stream,
                           nullptr, nullptr, slots);
}

extern "C" int vgr_foam_index_pack(const int32_t* offsets, const int32_t* nbr, const float* edge, const float* attr,
                                   int64_t n_sites, int64_t n_edges, float* edge_i, float* attr_i, void* stream) {
    VGR_REQUIRE(n_sites >= 0 && n_sites <= INT_MAX, "foam_index_pack: n_sites must be in [0, 2^31)");
    VGR_REQUIRE(n_edges >= n_sites && n_edges <= INT_MAX, "foam_index_pack: n_edges must be in [N, 2^31)");
    if (n_sites == 0) return VGR_OK;
    VGR_REQUIRE(offsets && nbr && edge && attr && edge_i && attr_i, "foam_index_pack: null pointer");
    const int64_t total = n_edges + 20 * n_sites;
    hipLaunchKernelGGL(vgr::index_pack_kernel, dim3(vgr::grid_for(total, 256)), dim3(256), 0, vgr::as_stream(stream),
                       offsets, nbr, reinterpret_cast<const float4*>(edge), attr, n_sites, n_edges,
                       reinterpret_cast<float4*>(edge_i), attr_i);
    return vgr::launch_status("index_pack_kernel");
}

extern "C" int vgr_foam_infer_indexed(const float* points, int64_t n_sites, const int32_t* offsets,
                                      const int32_t* nbr, const float* edge, int64_t n_edges, const float* attr,
                                      const void* sh, int32_t sh_half, int64_t sh_deg, const float* o, const float* d,
                                      const int32_t* start, const float* near_t, const float* far_t, int64_t n_rays,
                                      double t_thresh, double w_thresh, double color_cut, int64_t color_mode,
                                      int64_t stage, const int32_t* cap, const int32_t* orig, float* rgb, float* T,
                                      float* depth, int32_t* stats, int32_t* trace, int64_t trace_cap,
                                      const int32_t* order, int64_t lanes_per_ray, const float* edge_i,
                                      const float* attr_i, const int32_t* slots, const float* rows,
                                      int64_t row_floats, void* stream) {
    VGR_REQUIRE(trace == nullptr || trace_cap > 0, "foam_infer_indexed: trace needs trace_cap > 0");
    VGR_REQUIRE(edge_i && attr_i, "foam_infer_indexed: edge_i and attr_i are required");
    VGR_REQUIRE(rows == nullptr || reinterpret_cast<uintptr_t>(rows) % (row_floats == 64 ? 256 : 64) == 0,
                "foam_infer_indexed: rows must be 64-byte aligned, site blocks 256-byte aligned");
    return vgr::foam_entry(points, n_sites, offsets, nbr, edge, n_edges, attr, sh, sh_half, sh_deg, o, d, start,
                           near_t, far_t, n_rays, t_thresh, w_thresh, color_cut, color_mode, stage, cap, orig, rgb,
                           T, depth, stats, trace, trace == nullptr ? 0 : trace_cap, order, lanes_per_ray, stream,
                           edge_i, attr_i, slots, rows, row_floats);
}

extern "C" int vgr_foam_slot_table(const int32_t* offsets, const int32_t* nbr, int64_t n_sites, int64_t n_edges,
                                   int32_t* slots, void* stream) {
    VGR_REQUIRE(n_sites >= 0 && n_sites <= INT_MAX, "foam_slot_table: n_sites must be in [0, 2^31)");
    VGR_REQUIRE(n_edges >= n_sites && n_edges <= INT_MAX, "foam_slot_table: n_edges must be in [N, 2^31)");
    if (n_sites == 0) return VGR_OK;
    VGR_REQUIRE(offsets && nbr && slots, "foam_slot_table: null pointer");
    VGR_REQUIRE(reinterpret_cast<uintptr_t>(slots) % 16 == 0, "foam_slot_table: slots must be 16-byte aligned");
    hipLaunchKernelGGL(vgr::slot_table_kernel, dim3(vgr::grid_for(n_sites, 256)), dim3(256), 0, vgr::as_stream(stream),
                       offsets, nbr, n_sites, reinterpret_cast<int4*>(slots));
    return vgr::launch_status("slot_table_kernel");
}
