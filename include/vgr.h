/*
 * vgr -- MI355X-native (gfx950) forward/inference renderer of the voronoi-gauss field.
 *
 * C ABI of libvgr.so. Every entry point takes raw device pointers (inputs borrowed for the duration of the
 * asynchronous launch, outputs owned and allocated by the caller), element counts, and the HIP stream as an
 * opaque pointer (NULL = the default stream). Launches are asynchronous: nothing here synchronises.
 * Return value: VGR_OK, or an error code with a message available from vgr_last_error() (thread-local).
 * A count of zero rays / samples / sites is valid and launches nothing, like the reference (outputs untouched).
 *
 * Arrays are C-contiguous. Shapes use N sites, E = sum of self-inclusive neighbourhood sizes, M = E - N,
 * B rays, S samples per ray, m samples.
 */
#ifndef VGR_H
#define VGR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VGR_OK 0
#define VGR_ERR_INVALID 1 /* bad argument: null pointer, size, mode out of range */
#define VGR_ERR_LAUNCH 2  /* the HIP runtime reported a launch or device error */

#define VGR_COLOR_LAZY 0  /* "exact": colours in a second pass for segments with weight > w_thresh */
#define VGR_COLOR_BAKED 1 /* per-view site colours stored in attr[:, 16:19] */
#define VGR_COLOR_FUSED 2 /* online blend in the density pass */

/* Message of the last failing call on this thread ("" if none). */
const char* vgr_last_error(void);

/* ABI version of this library (incremented on any signature change). */
int vgr_abi_version(void);

/*
 * Inference rendering at the ray / Voronoi-face interaction points (thread per ray, wave64 tiles).
 * Replaces foam_infer() of csrc/foam_infer.cu:376-435 (pybind11 export :437-440), bound by
 * ext.foam_infer_extension() (ext.py:42-43) and called from render_rays_foam_infer (render.py:251-255).
 *
 *   points  f32 (N, 4)            site positions (4th component unused)
 *   offsets i32 (N + 1)           self-first neighbourhood CSR (offsets[c] is the edge of c itself)
 *   nbr     i32 (E)               site of every edge
 *   edge    f32 (E, 4)            (p_j, half2(r2_j, lam_j) bit pattern)
 *   attr    f32 (N, 20)           dA(6), min(raw, 30), 0, cA(6), 0, 0, baked rgb(3), 0
 *   sh      f32 (N, 16, 3) or f16 (sh_half = 1); may be NULL in baked mode
 *   o, d    f32 (B, 3); start i32 (B); near_t, far_t f32 (B)
 *   cap     i32 (B) per-ray sample budget, or NULL (unbounded)
 *   orig    i32 (N) original site index for tie-breaking after a renumbering, or NULL
 *   outputs rgb f32 (B, 3) foreground (no background), T f32 (B), depth f32 (B),
 *           stats i32 (B, 5) = samples, segments with colour, walk steps, density terms, SH evaluations (the colour
 *           lookups that miss the reference's per-ray cache of 8 direct-mapped slots keyed by site & 7,
 *           csrc/foam_infer.cu:151-168; kept here as 8 tags per ray in LDS, checked at every lookup)
 * color_mode: VGR_COLOR_*; stage: 0 exit faces only, 1 + density, 2 full rendering.
 * Rays whose start index is outside [0, N) are not traced: rgb = depth = 0, T = 1, stats = 0.
 */
int vgr_foam_infer(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* nbr,
                   const float* edge, int64_t n_edges, const float* attr, const void* sh, int32_t sh_half,
                   int64_t sh_deg, const float* o, const float* d, const int32_t* start, const float* near_t,
                   const float* far_t, int64_t n_rays, double t_thresh, double w_thresh, double color_cut,
                   int64_t color_mode, int64_t stage, const int32_t* cap, const int32_t* orig, float* rgb,
                   float* T, float* depth, int32_t* stats, void* stream);

/*
 * vgr_foam_infer plus a trace sink: trace i32 (B, trace_cap) receives the cell of every sample, in original
 * numbering (orig[c] when orig is given), for the first min(stats[:, 0], trace_cap) samples of each ray.
 * No counterpart in the reference (it has no trace output); used to check visited-cell sequences.
 */
int vgr_foam_infer_traced(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* nbr,
                          const float* edge, int64_t n_edges, const float* attr, const void* sh, int32_t sh_half,
                          int64_t sh_deg, const float* o, const float* d, const int32_t* start, const float* near_t,
                          const float* far_t, int64_t n_rays, double t_thresh, double w_thresh, double color_cut,
                          int64_t color_mode, int64_t stage, const int32_t* cap, const int32_t* orig, float* rgb,
                          float* T, float* depth, int32_t* stats, int32_t* trace, int64_t trace_cap, void* stream);

/*
 * vgr_foam_infer_traced with the ray layout chosen by the caller: lanes_per_ray 1 runs one ray per lane, 2, 4 or 8
 * a group of that many lanes per ray (each lane takes every lanes_per_ray-th edge of a cell's neighbourhood; the
 * group combines exit faces by a lexicographic minimum, so the visited cells are the same, and density and colour
 * terms by sums, so only their summation order differs), 0 the library's default (the layout vgr_foam_infer runs:
 * 4 lanes per ray for stages 0 and 1 and lazy colours, one ray per lane for fused and baked colours). Fused and
 * baked colours with a finite color_cut always run one ray per lane (their neighbour skipping follows the edge
 * order). trace may be NULL (then trace_cap is ignored). order (NULL = the batch order): a permutation of
 * 0 .. B - 1 giving the order in which the rays are traced (vgr_ray_order); results are the same in any order, an
 * entry outside [0, B) is skipped. slots (NULL = none): the slot table of vgr_foam_slot_table for this pack; with
 * color_cut = +inf the reference's cache misses (stats[:, 4]) then come from it once per neighbourhood pass instead
 * of from per-lookup tags in LDS (same counts, less work). No counterpart in the reference: the layout comparison
 * for vgr_foam_infer, whose arguments and outputs it otherwise shares.
 */
int vgr_foam_infer_lanes(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* nbr,
                         const float* edge, int64_t n_edges, const float* attr, const void* sh, int32_t sh_half,
                         int64_t sh_deg, const float* o, const float* d, const int32_t* start, const float* near_t,
                         const float* far_t, int64_t n_rays, double t_thresh, double w_thresh, double color_cut,
                         int64_t color_mode, int64_t stage, const int32_t* cap, const int32_t* orig, float* rgb,
                         float* T, float* depth, int32_t* stats, int32_t* trace, int64_t trace_cap,
                         const int32_t* order, int64_t lanes_per_ray, const int32_t* slots, void* stream);

/*
 * Cell traversal alone (foam_infer with stage 0: walk to the start cell, then exit faces up to far or cap) with a
 * group of lanes_per_ray lanes (4, 8 or 16; 0 = 4) per ray, each testing every lanes_per_ray-th face, and a group
 * min-reduction of the exit parameter. No counterpart in the reference: it is the lane-per-face layout against
 * which vgr_foam_infer's thread-per-ray layout is compared (same outputs bit for bit). stats i32 (B, 5) as
 * vgr_foam_infer's (sample and walk-step counts, the rest 0); trace (optional, NULL = none) i32 (B, trace_cap):
 * the cell of every sample in original numbering.
 */
int vgr_foam_traverse_faces(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* nbr,
                            const float* edge, int64_t n_edges, const float* o, const float* d, const int32_t* start,
                            const float* near_t, const float* far_t, int64_t n_rays, const int32_t* cap,
                            const int32_t* orig, int32_t* stats, int32_t* trace, int64_t trace_cap,
                            int64_t lanes_per_ray, void* stream);

/*
 * Fused uniform-step march (forward). Replaces march_forward() of csrc/march.cu:383-403 (export :432),
 * bound by ext.march (ext.py:172-182) and called from render_rays_uniform (render.py:118-119).
 *   points f32 (N, 3), offsets i32 (N + 1), adj i32 (M) Delaunay CSR; raw f32 (N); dA, cA f32 (N, 6) conics;
 *   sh f32 (N, 16, 3); o, d f32 (B, 3); start i32 (B); near_t, mid_t, far_t f32 (B)
 *   outputs rgb f32 (B, 3), T f32 (B), depth f32 (B), stats i32 (B, 3) = samples, samples with colour, walk steps
 * trace (optional, NULL = none) i32 (B, trace_cap): the site of every sample.
 * work: device scratch of at least vgr_march_work_size(N, sh_deg) bytes (128 or 256 per site), 256-byte aligned,
 * for the packed site blocks (overwritten by every call; calls that share it must be ordered on one stream).
 */
int64_t vgr_march_work_size(int64_t n_sites, int64_t sh_deg);
int vgr_march_forward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                      int64_t n_adj, const float* raw, const float* dA, const float* cA, const float* sh,
                      int64_t sh_deg, const float* o, const float* d, const int32_t* start, const float* near_t,
                      const float* mid_t, const float* far_t, int64_t n_rays, double dt, int64_t n_bg,
                      double t_thresh, double w_thresh, float* rgb, float* T, float* depth, int32_t* stats,
                      int32_t* trace, int64_t trace_cap, void* work, int64_t work_bytes, void* stream);

/*
 * vgr_march_forward with the ray layout chosen by the caller: lanes_per_ray 1 (one ray per lane), 16 (a group of
 * 16 lanes per ray, one neighbour per lane: for small batches, whose launches are bound by each ray's serial chain
 * of loads) or 0 (by batch size: 16 below 524288 rays, else 1, which is what vgr_march_forward does). The layouts
 * visit the same sites; their sums differ in the order of addition. order (NULL = the batch order): the order in
 * which the rays are traced, as for vgr_foam_infer_lanes. Same reference function as vgr_march_forward.
 */
int vgr_march_forward_lanes(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                            int64_t n_adj, const float* raw, const float* dA, const float* cA, const float* sh,
                            int64_t sh_deg, const float* o, const float* d, const int32_t* start,
                            const float* near_t, const float* mid_t, const float* far_t, int64_t n_rays, double dt,
                            int64_t n_bg, double t_thresh, double w_thresh, float* rgb, float* T, float* depth,
                            int32_t* stats, int32_t* trace, int64_t trace_cap, const int32_t* order,
                            int64_t lanes_per_ray, void* work, int64_t work_bytes, void* stream);

/*
 * Fused uniform-step march (backward: re-marches every ray). Replaces march_backward() of csrc/march.cu:405-428
 * (kernel :264-345, export :433), called by _March.backward (ext.py:162-169) when training through ext.march.
 *   The field, rays and march parameters are the forward's; rgb f32 (B, 3) and T f32 (B) are the forward's outputs
 *   and g_rgb f32 (B, 3), g_T f32 (B) their upstream gradients.
 *   -> g_raw f32 (N), g_dA f32 (N, 6), g_cA f32 (N, 6), g_sh f32 (N, 16, 3), overwritten (zeroed first). The sums
 *   use fp32 atomics, so they agree with a sequential sum to rounding, not bitwise.
 * lanes_per_ray: the forward's layout (0, 1 or 16 as for vgr_march_forward_lanes); it must be the one that produced
 * rgb and T, since the backward replays that forward's sums. blocks_ready: nonzero when `work` is the forward's
 * workspace, still holding the site blocks it packed from these same field arrays (the pack is then skipped).
 * work: device scratch of vgr_march_backward_work_size(N, sh_deg) bytes (the forward's site blocks plus a 256-byte
 * gradient block per site), 256-byte aligned.
 */
int64_t vgr_march_backward_work_size(int64_t n_sites, int64_t sh_deg);
int vgr_march_backward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                       int64_t n_adj, const float* raw, const float* dA, const float* cA, const float* sh,
                       int64_t sh_deg, const float* o, const float* d, const int32_t* start, const float* near_t,
                       const float* mid_t, const float* far_t, int64_t n_rays, double dt, int64_t n_bg,
                       double t_thresh, double w_thresh, const float* rgb, const float* T, const float* g_rgb,
                       const float* g_T, float* g_raw, float* g_dA, float* g_cA, float* g_sh, int64_t lanes_per_ray,
                       int64_t blocks_ready, void* work, int64_t work_bytes, void* stream);

/*
 * The training renderer: rendering at the ray's crossings of the Voronoi faces with a record of every sample, and
 * its backward. Replaces foam_forward() / foam_backward() of csrc/foam.cu:471-531 (kernels :345-469, exports
 * :533-536), bound by ext.foam (ext.py:185-216), the renderer train.py uses by default (render_rays_foam).
 * Both run 16 lanes per ray (one neighbour per lane), the layout for training batches.
 *   Field and rays as for vgr_march_forward (no mid_t). foam_forward -> rgb f32 (B, 3), T f32 (B), depth f32 (B),
 *   stats i32 (B, 3) = samples, coloured segments, walk steps; rec f32 (B, record_cap, 8) = per sample (t, site
 *   bits, sigma, C rgb, m_min, 1 / sum of colour weights or 0) for the first record_cap samples (record_cap 0: no
 *   records, rec may be NULL).
 *   foam_backward takes the forward's rgb, T, rec and stats (records replayed for rays whose samples fit, the others
 *   re-traced with the same arithmetic) and the upstream gradients g_rgb (B, 3), g_T (B) -> g_raw (N), g_dA (N, 6),
 *   g_cA (N, 6), g_sh (N, 16, 3), overwritten. Sums use fp32 atomics (equal to a sequential sum to rounding).
 * work: vgr_foam_work_size(N, sh_deg) bytes, 256-byte aligned, for both; blocks_ready as for vgr_march_backward
 * (nonzero: `work` is the forward's, whose site blocks are reused).
 */
int64_t vgr_foam_work_size(int64_t n_sites, int64_t sh_deg);
int vgr_foam_forward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj, int64_t n_adj,
                     const float* raw, const float* dA, const float* cA, const float* sh, int64_t sh_deg,
                     const float* o, const float* d, const int32_t* start, const float* near_t, const float* far_t,
                     int64_t n_rays, double t_thresh, double w_thresh, float* rgb, float* T, float* depth,
                     int32_t* stats, float* rec, int64_t record_cap, void* work, int64_t work_bytes, void* stream);
int vgr_foam_backward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                      int64_t n_adj, const float* raw, const float* dA, const float* cA, const float* sh,
                      int64_t sh_deg, const float* o, const float* d, const int32_t* start, const float* near_t,
                      const float* far_t, int64_t n_rays, double t_thresh, double w_thresh, const float* rgb,
                      const float* T, const float* g_rgb, const float* g_T, const float* rec, int64_t record_cap,
                      const int32_t* stats, float* g_raw, float* g_dA, float* g_cA, float* g_sh,
                      int64_t blocks_ready, void* work, int64_t work_bytes, void* stream);

/*
 * Nearest site of every sorted ray sample o + z d by a greedy walk (strict <). Replaces walk() of
 * csrc/vgf.cu:438-456 (export :566), bound by Graph.walk (ext.py:54-58).
 *   z f32 (B, S) sorted per ray; start i32 (B) -> site i32 (B, S), steps i32 (B) (steps may be NULL)
 */
int vgr_walk(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj, int64_t n_adj,
             const float* o, const float* d, const float* z, const int32_t* start, int64_t n_rays, int64_t n_samples,
             int32_t* site, int32_t* steps, void* stream);

/*
 * sigma(x) over the Voronoi neighbourhood of site. Replaces density_forward() of csrc/vgf.cu:458-475
 * (export :567), bound by ext.density (ext.py:78-87).
 *   raw f32 (N), log_scale f32 (N, 3), quat f32 (N, 4) wxyz; x f32 (m, 3), site i32 (m) -> sigma f32 (m)
 */
int vgr_density_forward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                        int64_t n_adj, const float* raw, const float* log_scale, const float* quat, const float* x,
                        const int32_t* site, int64_t m, double scale_mult, float* sigma, void* work,
                        int64_t work_bytes, void* stream);

/*
 * Normalised blend of max(SH_k(d) + 1/2, 0) over the Voronoi neighbourhood of site. Replaces color_forward()
 * of csrc/vgf.cu:494-513 (export :569), bound by ext.color (ext.py:108-117).
 *   log_scale f32 (N, 3), quat f32 (N, 4), sh f32 (N, 16, 3); x, dirs f32 (m, 3), site i32 (m) -> rgb f32 (m, 3)
 */
int vgr_color_forward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                      int64_t n_adj, const float* log_scale, const float* quat, const float* sh, int64_t sh_deg,
                      const float* x, const float* dirs, const int32_t* site, int64_t m, float* rgb, void* work,
                      int64_t work_bytes, void* stream);

/*
 * Optional device scratch of vgr_density_forward and vgr_color_forward (work may be NULL): with at least
 * vgr_field_work_size(N) bytes (16-byte aligned) and m >= N / 8 samples, the Gaussian of every site is built once per
 * call (rotation rows and inverse variances, the arithmetic each neighbour would repeat) and the per-sample kernels
 * read it; results are bit-identical either way. Calls sharing one work buffer must be ordered on one stream.
 */
int64_t vgr_field_work_size(int64_t n_sites);

/*
 * Conics A = R diag(1 / (s^2 + floor^2)) R^T as (xx, xy, xz, yy, yz, zz). Replaces conic_forward() of
 * csrc/vgf.cu:535-546 (export :564), bound by ext.conic (ext.py:134-136).
 *   log_scale f32 (n, 3), quat f32 (n, 4) -> A f32 (n, 6)
 */
int vgr_conic_forward(const float* log_scale, const float* quat, int64_t n, double floor, float* A, void* stream);

/*
 * Gradients of vgr_density_forward (scale_mult 1) for dL/dsigma = grad_sigma (m). Replaces density_backward() of
 * csrc/vgf.cu:477-492 (export :568), bound by ext._Density.backward (ext.py:69-75). Accumulated into g_raw (N),
 * g_ls (N, 3) and g_quat (N, 4), which the caller zeroes; terms with rho_k G_k |dL/dsigma| <= 1e-12 are skipped.
 * work: NULL (the per-site sums are scattered with fp32 atomics, one sample per lane), or device scratch of
 * vgr_density_backward_work_size(N, m) bytes, 256-byte aligned, with which the samples are counting-sorted by site
 * and each site gathers its gradients from the samples of its own and its neighbours' cells (no atomics on the
 * gradients). Either way the summation order, and so the last bits, vary from run to run. Calls sharing a
 * workspace must be ordered on one stream.
 */
int64_t vgr_density_backward_work_size(int64_t n_sites, int64_t m);
int vgr_density_backward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                         int64_t n_adj, const float* raw, const float* log_scale, const float* quat, const float* x,
                         const int32_t* site, int64_t m, const float* grad_sigma, float* g_raw, float* g_ls,
                         float* g_quat, void* work, int64_t work_bytes, void* stream);

/*
 * Gradients of vgr_color_forward for dL/drgb = grad_rgb (m, 3), given its output rgb (m, 3). Replaces
 * color_backward() of csrc/vgf.cu:515-533 (export :570), bound by ext._Color.backward (ext.py:99-105).
 * Accumulated into g_ls (N, 3), g_quat (N, 4) and g_sh (N, 16, 3), which the caller zeroes; normalised weights below
 * 1e-7 get no gradient. work: NULL (fp32 atomics) or the gather's scratch, as vgr_density_backward, of
 * vgr_color_backward_work_size(N, m) bytes.
 */
int64_t vgr_color_backward_work_size(int64_t n_sites, int64_t m);
int vgr_color_backward(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj,
                       int64_t n_adj, const float* log_scale, const float* quat, const float* sh, int64_t sh_deg,
                       const float* x, const float* dirs, const int32_t* site, int64_t m, const float* rgb,
                       const float* grad_rgb, float* g_ls, float* g_quat, float* g_sh, void* work,
                       int64_t work_bytes, void* stream);

/*
 * Gradients of vgr_conic_forward for dL/dA = gA (n, 6) (off-diagonal entries standing for both A_ab and A_ba),
 * written to g_ls (n, 3) and g_quat (n, 4). Replaces conic_backward() of csrc/vgf.cu:548-560 (export :565),
 * bound by ext._Conic.backward (ext.py:127-131).
 */
int vgr_conic_backward(const float* log_scale, const float* quat, int64_t n, double floor, const float* gA,
                       float* g_ls, float* g_quat, void* stream);

/*
 * The inference records of foam_infer from the model's tensors. Replaces the body of pack_foam()
 * (render.py:179-225, called by bench_infer.py:37-41 and eval_scene.py:69 before rendering).
 *   points f32 (N, 3), offsets i32 (N + 1), adj i32 (M): the Delaunay CSR; raw f32 (N); d_log_scale, c_log_scale
 *   f32 (N, 3); dA, cA f32 (N, 6) conics (vgr_conic_forward with scale_floor); sh f32 (N, 16, 3); perm i32 (N)
 *   new -> old renumbering (render.py:168-176) or NULL for none.
 *   -> points4 f32 (N, 4), offsets_sf i32 (N + 1) self-first, nbr i32 (M + N), edge f32 (M + N, 4) =
 *   (p_j, half2(r2_j, lam_j) bits), attr f32 (N, 20), sh32 f32 (N, 16, 3), sh16 (optional, NULL = none) f16
 *   (N, 16, 3); all in the new numbering. work: device scratch of vgr_pack_work_size(N) bytes, 256-byte aligned.
 */
int64_t vgr_pack_work_size(int64_t n_sites);

/*
 * Z-order keys of points f32 (n, 3) over their bounding box, bits per axis (<= 21): the keys morton_order()
 * (render.py:168-176) sorts to renumber the sites, with its arithmetic (q = trunc((p - lo) / max(hi - lo, 1e-12) *
 * (2^bits - 1)), bit b of axis a at bit 3 b + a) -> code i64 (n). work: vgr_morton_work_size(n) bytes.
 */
int64_t vgr_morton_work_size(int64_t n);
int vgr_morton_codes(const float* points, int64_t n, int32_t bits, int64_t* code, void* work, int64_t work_bytes,
                     void* stream);
/*
 * Per-view site colours for the baked colour mode: for every packed site i, max(SH_i(d_i) + 1/2, 0) with
 * d_i = normalize(p_i - (cx, cy, cz)) (norm clamped at 1e-12), written into attr[i, 16..18]. Replaces the torch
 * ops of the reference's baking step (render.py:228-235, run per camera before render_rays_foam_infer with
 * colors='baked'). points4 f32 (N, 4) and sh32 f32 (N, 16, 3) are vgr_pack_foam's outputs; attr f32 (N, 20).
 */
int vgr_bake_colors(const float* points4, const float* sh32, int64_t n_sites, int64_t sh_deg, double cx, double cy,
                    double cz, float* attr, void* stream);
int vgr_pack_foam(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* adj, int64_t n_adj,
                  const float* raw, const float* d_log_scale, const float* c_log_scale, const float* dA,
                  const float* cA, const float* sh, const int32_t* perm, double scale_floor, double eps_density,
                  float* points4, int32_t* offsets_sf, int32_t* nbr, float* edge, float* attr, float* sh32,
                  void* sh16, void* work, int64_t work_bytes, void* stream);

/*
 * Uniform grid over the sites for exact nearest-site queries: the start-cell locator. No kernel of the reference
 * corresponds; it replaces the host-side cKDTree query of nearest_sites() (sites.py:38-39), which finds the start
 * site per camera centre (bench_infer.py:60, eval_scene.py:69, bench_fps.py:156) and per ray origin of a ray batch.
 * Grid: res[0] x res[1] x res[2] cells of edge cell[a] from lo (host arrays of 3); cell (x, y, z) has index
 * (z res[1] + y) res[0] + x, G = res[0] res[1] res[2] <= 4096^2.
 *   points f32 (N, stride), xyz first; cell_start i32 (G + 1) and cell_sites i32 (N): the sites of cell g are
 *   cell_sites[cell_start[g] .. cell_start[g + 1]), in no particular order; work i32 (vgr_grid_work_size(N, G)).
 */
int64_t vgr_grid_work_size(int64_t n_sites, int64_t n_cells);
int vgr_grid_build(const float* points, int64_t n_sites, int32_t stride, const float* lo, const float* cell,
                   const int32_t* res, int32_t* cell_start, int32_t* cell_sites, int32_t* work, void* stream);

/*
 * Coherent processing order of a ray batch, for the `order` argument of vgr_foam_infer_lanes and
 * vgr_march_forward_lanes. No counterpart in the reference, which traces rays in the order given (config 5's
 * incoherent batch: origins uniform in a cube, directions uniform on the sphere). A permutation sorting the rays
 * by the octahedral bin of the direction on a dir_res x dir_res map (1..64), then by the Z-order of the origin with
 * pos_bits (1..10) bits per axis over the origins' bounding box (2 log2(dir_res) + 3 pos_bits <= 32 key bits).
 *   o, d f32 (B, 3) -> order i32 (B); work: vgr_ray_order_work_size(B) bytes, 256-byte aligned.
 */
int64_t vgr_ray_order_work_size(int64_t n_rays);
int vgr_ray_order(const float* o, const float* d, int64_t n_rays, int32_t dir_res, int32_t pos_bits, int32_t* order,
                  void* work, int64_t work_bytes, void* stream);

/*
 * Indexed edge records of a foam pack, for vgr_foam_infer_indexed. No counterpart in the reference, whose kernel
 * reads two streams per neighbourhood entry (the float4 record and the int neighbour index, csrc/foam_infer.cu:
 * 183-184, 212-213, 269-272). This layout carries both in one record: edge_i[e] = (p_j, the bits of j = nbr[e])
 * and attr_i = attr with column 7 (zero padding in the reference layout) holding the bits of site k's cut-off word
 * half2(r2_k, lam_k), which every record pointing at k carries in edge[:, 3] (the self entry's, edge[offsets[k]]).
 *   offsets i32 (N + 1), nbr i32 (E), edge f32 (E, 4), attr f32 (N, 20) as for vgr_foam_infer
 *   -> edge_i f32 (E, 4), attr_i f32 (N, 20); a snapshot: rebuild after changing the pack.
 */
int vgr_foam_index_pack(const int32_t* offsets, const int32_t* nbr, const float* edge, const float* attr,
                        int64_t n_sites, int64_t n_edges, float* edge_i, float* attr_i, void* stream);

/*
 * vgr_foam_infer_lanes with the indexed edge records of vgr_foam_index_pack: the full fused rendering (stage 2,
 * VGR_COLOR_FUSED) with one ray per lane (lanes_per_ray 0 or 1) reads edge_i and attr_i in place of nbr, edge and
 * attr, one record stream per neighbourhood entry instead of two. The outputs are bit-identical to
 * vgr_foam_infer_lanes on the same pack. Exact colours (VGR_COLOR_LAZY, stage 2) with one ray per lane, slots
 * given and color_cut +inf run as that same fused blend: rgb, T, depth and stats[:, 0..3] bit-identical to
 * VGR_COLOR_FUSED (rgb within rounding of the two-pass exact colour: the same normalised sum over every neighbour,
 * kept relative to a running minimum), stats[:, 4] the exact mode's cache misses (its colour passes: segments of
 * weight > w_thresh). Every other stage, colour mode or layout runs vgr_foam_infer_lanes on the reference records
 * unchanged. slots as for vgr_foam_infer_lanes. rows (NULL = none): site rows of row_floats floats each, the first
 * 16 being the first 16 columns of attr (density conic, min(raw, 30), the cut-off word or padding, colour conic),
 * which the group layouts (lanes_per_ray 2, 4, 8) with fused colours then read in place of the 80-byte attr rows
 * (bit-identical results). row_floats 16: f32 (N, 16), 64-byte aligned, two whole rows per 128-byte line, where
 * 3 in 8 attr rows straddle two lines. row_floats 64: 256-byte site blocks f32 (N, 64), 256-byte aligned, whose
 * last 48 floats are the site's fp32 SH row as in sh (sh_half must be 0); those kernels then read the SH rows
 * from the blocks too, so that a neighbour visit's record and SH row take two 128-byte lines instead of three.
 * No counterpart in the reference (same function as vgr_foam_infer).
 */
int vgr_foam_infer_indexed(const float* points, int64_t n_sites, const int32_t* offsets, const int32_t* nbr,
                           const float* edge, int64_t n_edges, const float* attr, const void* sh, int32_t sh_half,
                           int64_t sh_deg, const float* o, const float* d, const int32_t* start, const float* near_t,
                           const float* far_t, int64_t n_rays, double t_thresh, double w_thresh, double color_cut,
                           int64_t color_mode, int64_t stage, const int32_t* cap, const int32_t* orig, float* rgb,
                           float* T, float* depth, int32_t* stats, int32_t* trace, int64_t trace_cap,
                           const int32_t* order, int64_t lanes_per_ray, const float* edge_i, const float* attr_i,
                           const int32_t* slots, const float* rows, int64_t row_floats, void* stream);

/*
 * Slot table of a foam pack, for the `slots` argument of vgr_foam_infer_lanes and vgr_foam_infer_indexed. No
 * counterpart in the reference, which keeps its per-ray colour cache of 8 direct-mapped slots (site & 7) in shared
 * memory and counts the lookups that miss it (csrc/foam_infer.cu:151-168, 359-360). A neighbourhood pass that looks
 * up every entry of cell c (colour cut-off +inf) hits that cache only at the first entry of a slot, and leaves the
 * slot's last entry in it; the table holds both per site:
 *   offsets i32 (N + 1), nbr i32 (E) as for vgr_foam_infer
 *   -> slots i32 (N, 16), 16-byte aligned: for slots s = 0..7 of site k's self-first neighbourhood in CSR order, the
 *      first and the last entry (F_s, L_s) at columns 2s, 2s + 1, -2 for a slot without entries; a snapshot: rebuild
 *      after changing the pack.
 */
int vgr_foam_slot_table(const int32_t* offsets, const int32_t* nbr, int64_t n_sites, int64_t n_edges, int32_t* slots,
                        void* stream);

/*
 * vgr_grid_build without a workspace argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. The scratch
 * (the cell of every site, the per-cell counters, the scan's tile sums) is a static device array of
 * VGR_GRID_NOALLOC_MAX_WORK ints (64 MiB), one per GPU, held until the process ends; a build needing more than
 * that (vgr_grid_work_size(N, G) > VGR_GRID_NOALLOC_MAX_WORK) is rejected with VGR_ERR_INVALID. It calls no
 * hipMalloc/hipFree and clears its counters with a kernel. Every call on one GPU uses that GPU's one array: calls
 * that overlap on a GPU (other streams, other host threads) race and must be serialised by the caller. The device
 * current on the calling thread must be the stream's. The first call on each device looks the array's address up
 * (hipGetSymbolAddress): make it outside graph capture (a warm call); every later call only launches kernels on
 * `stream`, so it can be captured and replayed. Same arguments and outputs as vgr_grid_build otherwise.
 */
#define VGR_GRID_NOALLOC_MAX_WORK (1LL << 24)
int vgr_grid_build_noalloc(const float* points, int64_t n_sites, int32_t stride, const float* lo, const float* cell,
                           const int32_t* res, int32_t* cell_start, int32_t* cell_sites, void* stream);

/*
 * Nearest site of every query point: the lexicographic argmin of (float64 squared distance, site index), as
 * cKDTree (float64) answers it up to exact distance ties.
 *   queries f32 (m, 3) -> site i32 (m); the grid arguments as built by vgr_grid_build
 */
int vgr_grid_nearest(const float* points, int64_t n_sites, int32_t stride, const float* lo, const float* cell,
                     const int32_t* res, const int32_t* cell_start, const int32_t* cell_sites, const float* queries,
                     int64_t n_queries, int32_t* site, void* stream);

/*
 * A cell-ordered copy of the sites of a grid built by vgr_grid_build (or _noalloc), for vgr_grid_nearest_points:
 * cell_points[s] = (x, y, z, bits of cell_sites[s]), so that the sites of a cell, and of a row of cells, lie in
 * consecutive 16-byte records. A snapshot of the positions: build it again after moving the sites. No counterpart in
 * the reference (part of the same replacement of nearest_sites, sites.py:38-39).
 *   points f32 (N, stride), cell_sites i32 (N) -> cell_points f32 (N, 4), 16-byte aligned
 */
int vgr_grid_cell_points(const float* points, int64_t n_sites, int32_t stride, const int32_t* cell_sites,
                         float* cell_points, void* stream);

/*
 * vgr_grid_nearest over the cell-ordered copy of vgr_grid_cell_points: the same answers bit for bit, with the
 * candidate sites read in cell order instead of through their indices (one 128-byte line per candidate there).
 * order (NULL = 0 .. m - 1): a permutation of the queries, the order in which they are answered (a lane skips an
 * entry outside [0, m)); a spatially coherent one (vgr_ray_order over the queries with dir_res 1, a Z-order of the
 * points) lets the lanes of a wave share the cells they scan. The answers do not depend on it.
 *   cell_points f32 (N, 4), 16-byte aligned; queries f32 (m, 3); order i32 (m) or NULL -> site i32 (m)
 */
int vgr_grid_nearest_points(const float* cell_points, int64_t n_sites, const float* lo, const float* cell,
                            const int32_t* res, const int32_t* cell_start, const float* queries, int64_t n_queries,
                            const int32_t* order, int32_t* site, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VGR_H */
