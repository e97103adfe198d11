// Bounding box of a point set on the GPU: per-block boxes, then one block reduces them (min and max are exact in
// any order, so the box is the same bits however the blocks are scheduled). Shared by the pack (Z-order keys of
// the sites) and the ray ordering (Z-order keys of the ray origins).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vgr {
namespace {

constexpr int kBoxBlock = 256;

// Per-block bounding boxes of the points: box[6 * block .. + 6) = (min xyz, max xyz).
__global__ void __launch_bounds__(kBoxBlock)
    bbox_blocks_kernel(const float* __restrict__ points, int64_t n, float* __restrict__ box) {
    __shared__ float part[6][kBoxBlock];
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBoxBlock + threadIdx.x;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const float v = i < n ? points[3 * i + a] : points[0];
        part[a][threadIdx.x] = v, part[3 + a][threadIdx.x] = v;
    }
    __syncthreads();
    for (int off = kBoxBlock / 2; off > 0; off >>= 1) {
        if (static_cast<int>(threadIdx.x) < off) {
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                part[a][threadIdx.x] = fminf(part[a][threadIdx.x], part[a][threadIdx.x + off]);
                part[3 + a][threadIdx.x] = fmaxf(part[3 + a][threadIdx.x], part[3 + a][threadIdx.x + off]);
            }
        }
        __syncthreads();
    }
    if (threadIdx.x < 6) box[6 * int64_t(blockIdx.x) + threadIdx.x] = part[threadIdx.x][0];
}

// Reduces the per-block boxes in place into box[0 .. 6) (one block; min and max are exact in any order).
__global__ void __launch_bounds__(kBoxBlock) bbox_final_kernel(float* __restrict__ box, int64_t n_blocks) {
    __shared__ float part[6][kBoxBlock];
    float v[6];
#pragma unroll
    for (int a = 0; a < 6; ++a) v[a] = box[a];
    for (int64_t b = threadIdx.x; b < n_blocks; b += kBoxBlock) {
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            v[a] = fminf(v[a], box[6 * b + a]);
            v[3 + a] = fmaxf(v[3 + a], box[6 * b + 3 + a]);
        }
    }
#pragma unroll
    for (int a = 0; a < 6; ++a) part[a][threadIdx.x] = v[a];
    __syncthreads();
    for (int off = kBoxBlock / 2; off > 0; off >>= 1) {
        if (static_cast<int>(threadIdx.x) < off) {
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                part[a][threadIdx.x] = fminf(part[a][threadIdx.x], part[a][threadIdx.x + off]);
                part[3 + a][threadIdx.x] = fmaxf(part[3 + a][threadIdx.x], part[3 + a][threadIdx.x + off]);
            }
        }
        __syncthreads();
    }
    __syncthreads();
    if (threadIdx.x < 6) box[threadIdx.x] = part[threadIdx.x][0];
}

// Bounding box (min xyz, max xyz) of n points of 3 floats into box[0 .. 6); box holds 6 floats per block of
// kBoxBlock points (the per-block boxes, reduced in place).
inline void bounding_box(const float* points, int64_t n, float* box, hipStream_t s) {
    const unsigned blocks = static_cast<unsigned>((n + kBoxBlock - 1) / kBoxBlock);
    hipLaunchKernelGGL(bbox_blocks_kernel, dim3(blocks), dim3(kBoxBlock), 0, s, points, n, box);
    hipLaunchKernelGGL(bbox_final_kernel, dim3(1), dim3(kBoxBlock), 0, s, box, int64_t(blocks));
}

}  // namespace
}  // namespace vgr
