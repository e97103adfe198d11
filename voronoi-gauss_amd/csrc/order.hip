// Coherent processing order for batches of rays, gfx950.
//
// The renderers give every lane (or group of lanes) of a wave one ray, in the order of the batch. Camera rays in
// 8x8 pixel tiles keep a wave's rays together; an incoherent batch (config 5: origins uniform in a cube, directions
// uniform on the sphere) gives every lane its own cache lines, and the wave-shared SH cache of foam_infer almost
// never hits. vgr_ray_order returns a permutation that sorts the rays by (direction bin, Z-order of the origin):
// the rays of a wave then start close together and travel in similar directions. The renderers take it as their
// processing order; each ray's result is unchanged (its arithmetic does not depend on the other lanes), only the
// order in which rays are traced.
//
// No kernel of the reference corresponds: it traces rays in the order it is given them.
#include <rocprim/device/device_radix_sort.hpp>

#include "vgr_abi.h"
#include "vgr_bbox.h"
#include "vgr_device.h"

namespace vgr {
namespace {

constexpr int kBlock = 256;

// Spreads the low 10 bits of v so that bit i lands at bit 3 i.
__device__ __forceinline__ uint32_t spread3(uint32_t v) {
    v &= 0x3ffu;
    v = (v | (v << 16)) & 0x030000ffu;
    v = (v | (v << 8)) & 0x0300f00fu;
    v = (v | (v << 4)) & 0x030c30c3u;
    return (v | (v << 2)) & 0x09249249u;
}

// Bin of a direction on a res x res octahedral map of the sphere (the upper hemisphere maps to the inner diamond,
// the lower one is folded over its edges); 0 for a zero direction.
__device__ __forceinline__ uint32_t direction_bin(float x, float y, float z, int res) {
    const float a = fabsf(x) + fabsf(y) + fabsf(z);
    if (!(a > 0.f)) return 0u;
    float u = x / a, v = y / a;
    if (z < 0.f) {
        const float fu = (1.f - fabsf(v)) * copysignf(1.f, u), fv = (1.f - fabsf(u)) * copysignf(1.f, v);
        u = fu, v = fv;
    }
    const int iu = min(max(static_cast<int>((u + 1.f) * 0.5f * res), 0), res - 1);
    const int iv = min(max(static_cast<int>((v + 1.f) * 0.5f * res), 0), res - 1);
    return static_cast<uint32_t>(iu * res + iv);
}

// key = direction bin above the origin's Z-order code (pos_bits bits per axis over the origins' bounding box).
__global__ void __launch_bounds__(kBlock)
    order_keys_kernel(const float* __restrict__ o, const float* __restrict__ d, int64_t n,
                      const float* __restrict__ box, int dir_res, int pos_bits, uint32_t* __restrict__ key,
                      int32_t* __restrict__ idx) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    const float cells = static_cast<float>(1 << pos_bits);
    uint32_t code = 0u;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const float lo = box[a], ext = fmaxf(box[3 + a] - lo, 1e-30f);
        const int q = min(max(static_cast<int>((o[3 * i + a] - lo) / ext * cells), 0), (1 << pos_bits) - 1);
        code |= spread3(static_cast<uint32_t>(q)) << a;
    }
    key[i] = (direction_bin(d[3 * i], d[3 * i + 1], d[3 * i + 2], dir_res) << (3 * pos_bits)) | code;
    idx[i] = static_cast<int32_t>(i);
}

constexpr int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

int key_bits(int dir_res, int pos_bits) {
    int bits = 3 * pos_bits;
    for (int bins = dir_res * dir_res - 1; bins > 0; bins >>= 1) ++bits;
    return bits;
}

size_t sort_temp_bytes(int64_t n, int bits) {
    size_t bytes = 0;
    (void)rocprim::radix_sort_pairs(nullptr, bytes, static_cast<const uint32_t*>(nullptr), static_cast<uint32_t*>(nullptr),
                              static_cast<const int32_t*>(nullptr), static_cast<int32_t*>(nullptr),
                              static_cast<size_t>(n), 0u, static_cast<unsigned>(bits));
    return bytes;
}

// Workspace: per-block boxes (6 floats per block), keys in and out, indices in, the sort's temporary storage.
int64_t order_bytes(int64_t n) {
    return align256(4 * 6 * ((n + kBoxBlock - 1) / kBoxBlock)) + 2 * align256(4 * n) + align256(4 * n) +
           align256(static_cast<int64_t>(sort_temp_bytes(n, 32)));
}

}  // namespace
}  // namespace vgr

extern "C" int64_t vgr_ray_order_work_size(int64_t n_rays) { return n_rays > 0 ? vgr::order_bytes(n_rays) : 0; }

extern "C" int vgr_ray_order(const float* o, const float* d, int64_t n_rays, int32_t dir_res, int32_t pos_bits,
                             int32_t* order, void* work, int64_t work_bytes, void* stream) {
    using namespace vgr;
    VGR_REQUIRE(n_rays >= 0 && n_rays <= INT_MAX, "ray_order: n_rays must be in [0, 2^31) (got %lld)",
                static_cast<long long>(n_rays));
    VGR_REQUIRE(dir_res >= 1 && dir_res <= 64, "ray_order: dir_res must be in [1, 64] (got %d)", dir_res);
    VGR_REQUIRE(pos_bits >= 1 && pos_bits <= 10, "ray_order: pos_bits must be in [1, 10] (got %d)", pos_bits);
    const int bits = key_bits(dir_res, pos_bits);
    VGR_REQUIRE(bits <= 32, "ray_order: %d direction bins and %d bits per axis need %d key bits (at most 32)",
                dir_res * dir_res, pos_bits, bits);
    if (n_rays == 0) return VGR_OK;
    VGR_REQUIRE(o && d && order, "ray_order: null pointer");
    const int64_t need = order_bytes(n_rays);
    VGR_REQUIRE(work && work_bytes >= need, "ray_order: work must hold vgr_ray_order_work_size(n) = %lld bytes",
                static_cast<long long>(need));
    VGR_REQUIRE(reinterpret_cast<uintptr_t>(work) % 256 == 0, "ray_order: work must be 256-byte aligned");
    char* w = static_cast<char*>(work);
    float* box = reinterpret_cast<float*>(w);
    w += align256(4 * 6 * ((n_rays + kBoxBlock - 1) / kBoxBlock));
    uint32_t* key_in = reinterpret_cast<uint32_t*>(w);
    w += align256(4 * n_rays);
    uint32_t* key_out = reinterpret_cast<uint32_t*>(w);
    w += align256(4 * n_rays);
    int32_t* idx = reinterpret_cast<int32_t*>(w);
    w += align256(4 * n_rays);
    size_t temp = sort_temp_bytes(n_rays, bits);
    VGR_REQUIRE(static_cast<int64_t>(temp) <= need - (w - static_cast<char*>(work)),
                "ray_order: the sort needs %zu bytes of temporary storage beyond the workspace", temp);
    const hipStream_t s = as_stream(stream);
    bounding_box(o, n_rays, box, s);
    hipLaunchKernelGGL(order_keys_kernel, dim3(grid_for(n_rays, kBlock)), dim3(kBlock), 0, s, o, d, n_rays, box,
                       int(dir_res), int(pos_bits), key_in, idx);
    if (int rc = launch_status("order_keys_kernel")) return rc;
    if (rocprim::radix_sort_pairs(w, temp, key_in, key_out, idx, order, static_cast<size_t>(n_rays), 0u,
                                  static_cast<unsigned>(bits), s) != hipSuccess)
        return launch_status("ray_order radix sort");
    return launch_status("ray_order");
}
