// Device primitives shared by the vgr kernels (gfx950, wave64).
//
// Arithmetic contract: every translation unit is compiled with -ffp-contract=off and IEEE fp32 division, so
// the products and sums that decide a walk or an exit face are rounded exactly as written, the same way the
// CPU oracle rounds them. Two things differ from the oracle by ulps only: exp (device exp2-based, against the
// CPU's libm), and the field arithmetic of foam_infer.hip (density, colour, blend), which fuses chosen products
// and sums into explicit FMAs (fmaf). Neither decides which cell a ray enters next;
// both can move a weight or transmittance across a threshold (w_thresh, t_thresh) when it is within ulps of it.
#pragma once

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

namespace vgr {

constexpr float kInf = 3.402823466e38f;  // "no value yet" sentinel of the reference kernels (FLT_MAX)
constexpr int kWalkCap = 4096;           // safety bound on greedy-walk steps per walk
constexpr int kMaxCells = 8192;          // safety bound on cells traversed per ray
constexpr int kXcds = 8;                 // MI355X: 8 XCDs, workgroups dispatched round-robin over them

// exp(x) through the hardware exp2 (HIP's __expf).
__device__ __forceinline__ float fexp(float x) { return __expf(x); }

// Workgroup id remapped so that XCD k (which receives the dispatch ids k, k + 8, k + 16, ...) processes one
// contiguous range of logical blocks: neighbouring ray tiles then share that XCD's L2.
__device__ __forceinline__ int64_t xcd_block_id() {
    const int64_t nb = gridDim.x, bid = blockIdx.x;
    const int64_t per = nb / kXcds, rem = nb % kXcds;
    const int64_t xcd = bid % kXcds, idx = bid / kXcds;
    return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

// v^T A v for A = (xx, xy, xz, yy, yz, zz).
__device__ __forceinline__ float maha(float xx, float xy, float xz, float yy, float yz, float zz, float vx, float vy,
                                      float vz) {
    return xx * vx * vx + yy * vy * vy + zz * vz * vz + 2.f * (xy * vx * vy + xz * vx * vz + yz * vy * vz);
}

// DPP row permutations for reductions inside groups of 2, 4, 8 or 16 consecutive lanes: quad_perm [1,0,3,2] and
// [2,3,0,1] (xor 1, xor 2), row_half_mirror (i <-> 7 - i within 8 lanes) and row_mirror (i <-> 15 - i within 16).
// A butterfly over them with a commutative operation leaves the same bits in every lane of the group.
constexpr int kXor1 = 0xB1, kXor2 = 0x4E, kHalfMirror = 0x141, kMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ int row_perm(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ float row_perm(float v) {
    return __int_as_float(row_perm<CTRL>(__float_as_int(v)));
}

// Real spherical-harmonics basis up to degree 3 (3DGS constants and signs), zero beyond `deg`.
__device__ inline void sh_basis(float x, float y, float z, int deg, float (&b)[16]) {
    b[0] = 0.28209479177387814f;
#pragma unroll
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

// Number of float4 holding the first 3 (deg + 1)^2 fp32 coefficients of a site, and of fp16 ones (8 per float4).
__host__ __device__ constexpr int sh_vec4_f32(int deg) { return (3 * (deg + 1) * (deg + 1) + 3) / 4; }
__host__ __device__ constexpr int sh_vec4_f16(int deg) { return (3 * (deg + 1) * (deg + 1) + 7) / 8; }

}  // namespace vgr
