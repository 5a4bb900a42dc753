// Extended narrow phase on the GPU, batched one pair per lane (the device code is in
// narrow_ext.h). Each lane handles one pair: two 64-B operand records in, one 64-B result
// out, so a launch is a single streaming pass of 192 B of HBM traffic per pair.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "collide.h"
#include "narrow_ext.h"

namespace za {
namespace {
using namespace np;

// Each lane loads its own two operand records (consecutive lanes, consecutive 64-B records:
// the four 16-B loads of a wave cover whole cache lines between them). Results go through
// LDS so that each store instruction of a wave writes 1 KB of consecutive memory (lane l
// stores quads l, l + 64, l + 128, l + 192 of the wave's 4 KB block). 16 KB of LDS per
// 256-lane block leaves occupancy to the register budget.
constexpr int kCollideBlock = 256;
constexpr int kRecQuads = 4;  // 64-B records

__global__ __launch_bounds__(kCollideBlock) void detect_collisions_kernel(const ZenoAmdCollider* a, const ZenoAmdCollider* b,
                                                                          uint32_t n, ZenoAmdContactResult* out) {
    __shared__ float4 stage[kCollideBlock / 64][64 * kRecQuads];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const size_t base = (size_t)blockIdx.x * kCollideBlock + (size_t)wave * 64u;  // first pair of this wave
    const size_t i = base + lane;
    Result r = miss();
    if (i < n) r = detect(load_side(a + i), load_side(b + i));
    float4* so = stage[wave] + lane * kRecQuads;
    so[0] = make_float4(r.point.x, r.point.y, r.point.z, r.pen);
    so[1] = make_float4(r.normal.x, r.normal.y, r.normal.z, __uint_as_float(r.valid ? 1u : 0u));
    so[2] = make_float4(r.la.x, r.la.y, r.la.z, 0.0f);
    so[3] = make_float4(r.lb.x, r.lb.y, r.lb.z, 0.0f);
    __syncthreads();
    const size_t nq = (size_t)n * kRecQuads;
    float4* qo = reinterpret_cast<float4*>(out) + base * kRecQuads;
#pragma unroll
    for (int k = 0; k < kRecQuads; ++k) {
        const uint32_t q = lane + 64u * k;
        if (base * kRecQuads + q < nq) qo[q] = stage[wave][q];
    }
}

}  // namespace

hipError_t launch_detect_collisions(const ZenoAmdCollider* a, const ZenoAmdCollider* b, uint32_t n, ZenoAmdContactResult* out,
                                    hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const uint32_t blocks = (uint32_t)(((size_t)n + kCollideBlock - 1) / kCollideBlock);
    hipLaunchKernelGGL(detect_collisions_kernel, dim3(blocks), dim3(kCollideBlock), 0, stream, a, b, n, out);
    return hipGetLastError();
}

}  // namespace za
