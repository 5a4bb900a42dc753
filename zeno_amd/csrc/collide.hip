// Extended narrow phase on the GPU, batched one pair per lane (the device code is in
// narrow_ext.h). Each lane handles one pair: two 64-B operand records in, one 64-B result
// out, so a launch is a single streaming pass of 192 B of HBM traffic per pair.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstring>
#include <mutex>

#include "collide.h"
#include "narrow_ext.h"

namespace za {
namespace {
using namespace np;

// A block takes 256 consecutive pairs. A pair's geom types select one of detect()'s branches
// and a wave runs every branch its lanes need, so a mixed batch would pay for most of them in
// every wave. Each lane loads its own pair's two 64-B records (consecutive lanes, consecutive
// records: one streaming pass), and the block orders its pairs by ordered type pair (64
// classes), stably: each wave counts its lanes class by class with ballots (one round per
// class present in the wave), the counts are scanned over (class, wave), and lane t then
// evaluates the pair at position t of that order. The records move to their new lanes
// through one 16 KB LDS buffer, operand a then operand b (column-major: quad k of pair p at
// k * 256 + p, so the lanes' 16-B accesses of one quad are consecutive). A block of one type
// pair (every lane's class equal to lane 0's) skips the ordering and the exchange. Every record is read from HBM once. Each
// pair's result depends on that pair alone, so the order changes no result. Results go
// through the same buffer at the pair's own position, so that each store instruction of a
// wave writes 1 KB of consecutive memory (lane l stores quads l, l + 64, l + 128, l + 192 of
// its wave's 4 KB block).
constexpr int kCollideBlock = 256;
constexpr int kCollideWaves = kCollideBlock / 64;
constexpr int kRecQuads = 4;  // 64-B records
constexpr uint32_t kClasses = 64;

__global__ __launch_bounds__(kCollideBlock) void detect_collisions_kernel(const ZenoAmdCollider* a, const ZenoAmdCollider* b,
                                                                          uint32_t n, ZenoAmdContactResult* out) {
    __shared__ float4 stage[kCollideBlock * kRecQuads];   // 16 KB: operand exchange, then results
    __shared__ uint32_t wcount[kCollideWaves][kClasses];  // lanes of each class per wave, then offsets
    __shared__ uint16_t order[kCollideBlock];
    __shared__ uint32_t cls0;
    const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63u;
    const size_t blk = (size_t)blockIdx.x * kCollideBlock;
    const size_t i = blk + t;
    wcount[wave][lane] = 0u;
    float4 q[2 * kRecQuads];
#pragma unroll
    for (int k = 0; k < 2 * kRecQuads; ++k) q[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    uint32_t cls = kClasses - 1u;  // lanes past the end: the last class, evaluated as nothing
    if (i < n) {
        const float4* pa = reinterpret_cast<const float4*>(a + i);
        const float4* pb = reinterpret_cast<const float4*>(b + i);
#pragma unroll
        for (int k = 0; k < kRecQuads; ++k) { q[k] = pa[k]; q[kRecQuads + k] = pb[k]; }
        cls = (__float_as_uint(q[0].x) & 7u) * 8u + (__float_as_uint(q[kRecQuads].x) & 7u);
    }
    if (t == 0) cls0 = cls;
    __syncthreads();
    uint32_t src = t;
    if (!__syncthreads_and(cls == cls0)) {
        uint32_t rank = 0;  // position among the wave's lanes of this class
        uint64_t pending = __ballot(1);
        while (pending) {
            const int leader = __ffsll((unsigned long long)pending) - 1;
            const uint32_t c = __shfl(cls, leader);
            const uint64_t same = __ballot(cls == c);
            if ((int)lane == leader) wcount[wave][c] = (uint32_t)__popcll(same);
            if (cls == c) rank = (uint32_t)__popcll(same & ((1ull << lane) - 1ull));
            pending &= ~same;
        }
        __syncthreads();
        if (wave == 0) {  // offsets in (class, wave) order: lane c scans class c's total
            uint32_t cnt[kCollideWaves];
            uint32_t tot = 0;
#pragma unroll
            for (int w = 0; w < kCollideWaves; ++w) { cnt[w] = wcount[w][lane]; tot += cnt[w]; }
            uint32_t incl = tot;
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t x = __shfl_up(incl, d);
                if ((int)lane >= d) incl += x;
            }
            uint32_t run = incl - tot;
#pragma unroll
            for (int w = 0; w < kCollideWaves; ++w) { wcount[w][lane] = run; run += cnt[w]; }
        }
        __syncthreads();
        order[wcount[wave][cls] + rank] = (uint16_t)t;
        __syncthreads();
        src = order[t];
#pragma unroll
        for (int h = 0; h < 2; ++h) {  // operand a, then operand b
#pragma unroll
            for (int k = 0; k < kRecQuads; ++k) stage[k * kCollideBlock + t] = q[h * kRecQuads + k];
            __syncthreads();
#pragma unroll
            for (int k = 0; k < kRecQuads; ++k) q[h * kRecQuads + k] = stage[k * kCollideBlock + src];
            __syncthreads();
        }
    }
    Result r = miss();
    if (blk + src < n) r = detect(side_from(q[0], q[1], q[2], q[3]), side_from(q[4], q[5], q[6], q[7]));
    float4* so = stage + src * kRecQuads;
    so[0] = make_float4(r.point.x, r.point.y, r.point.z, r.pen);
    so[1] = make_float4(r.normal.x, r.normal.y, r.normal.z, __uint_as_float(r.valid ? 1u : 0u));
    so[2] = make_float4(r.la.x, r.la.y, r.la.z, 0.0f);
    so[3] = make_float4(r.lb.x, r.lb.y, r.lb.z, 0.0f);
    __syncthreads();
    const size_t base = blk + (size_t)wave * 64u;  // first pair of this wave's store block
    const size_t nq = (size_t)n * kRecQuads;
    float4* qo = reinterpret_cast<float4*>(out) + base * kRecQuads;
    const float4* sw = stage + wave * 64u * kRecQuads;
#pragma unroll
    for (int k = 0; k < kRecQuads; ++k) {
        const uint32_t qq = lane + 64u * k;
        if (base * kRecQuads + qq < nq) qo[qq] = sw[qq];
    }
}

// Staging of zeno_amd_detect_collisions_host_noalloc: operands a, operands b and results of
// up to ZENO_AMD_NOALLOC_MAX_PAIRS pairs (64 B each, 3 MiB in all). Every GPU the library runs
// on holds its own copy until the process ends, and every call on that GPU shares it. In host
// code `scratch` names a host-side stand-in: its device address on each GPU comes from
// hipGetSymbolAddress (scratch_on_current_device) and only that address reaches a kernel or
// a copy.
constexpr size_t kNoAllocPairs = ZENO_AMD_NOALLOC_MAX_PAIRS;
constexpr size_t kNoAllocBytes = kNoAllocPairs * (2 * sizeof(ZenoAmdCollider) + sizeof(ZenoAmdContactResult));
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

constexpr int kMaxDevices = 64;

// One lock per device: a call holds its device's lock from the first copy into `scratch`
// until its results are back, so calls from several host threads on one GPU take turns.
std::mutex device_lock[kMaxDevices];

// Device address of `scratch` on the current device (looked up once per device with that
// device current) and the device's index.
hipError_t scratch_on_current_device(unsigned char** out, int* device) {
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        addr[dev] = p;
    }
    *out = static_cast<unsigned char*>(addr[dev]);
    *device = dev;
    return hipSuccess;
}

}  // namespace

hipError_t detect_collisions_host_noalloc(const ZenoAmdCollider* a, const ZenoAmdCollider* b, uint32_t n,
                                          ZenoAmdContactResult* out) {
    if (n == 0) return hipSuccess;
    if (n > kNoAllocPairs) return hipErrorInvalidValue;
    unsigned char* base = nullptr;
    int dev = 0;
    hipError_t e = scratch_on_current_device(&base, &dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> hold(device_lock[dev]);
    ZenoAmdCollider* da = reinterpret_cast<ZenoAmdCollider*>(base);
    ZenoAmdCollider* db = da + kNoAllocPairs;
    ZenoAmdContactResult* dout = reinterpret_cast<ZenoAmdContactResult*>(db + kNoAllocPairs);
    const size_t in_bytes = (size_t)n * sizeof(ZenoAmdCollider), out_bytes = (size_t)n * sizeof(ZenoAmdContactResult);
    // The null stream orders the copies and the kernel; the kernel writes every result of
    // the n pairs, so nothing left in the array by an earlier call is read.
    if ((e = hipMemcpy(da, a, in_bytes, hipMemcpyHostToDevice)) != hipSuccess) return e;
    if ((e = hipMemcpy(db, b, in_bytes, hipMemcpyHostToDevice)) != hipSuccess) return e;
    if ((e = launch_detect_collisions(da, db, n, dout, nullptr)) != hipSuccess) return e;
    return hipMemcpy(out, dout, out_bytes, hipMemcpyDeviceToHost);
}

namespace {
__global__ __launch_bounds__(256) void selfcheck_divide_kernel(const float* a, const float* b, float* q, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    // The step kernel's four-quotient path (qdivs), with neighbouring lanes of the operand.
    if (i < n) q[i] = qdivs(q4{a[i], 0.0f, -a[i], a[i]}, b[i]).w;
}
// max |1 - b rcp64(b)| over the fp32 bit patterns [base, base + 2^32 / gridDim.x ...): each
// thread takes 256 consecutive patterns; a wave reduces its lanes and one lane folds the wave's
// maximum into *out with a vector atomic (non-negative doubles order as their bit patterns).
__global__ __launch_bounds__(256) void selfcheck_rcp_error_kernel(unsigned long long* out) {
    const uint64_t base = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 256ull;
    double m = 0.0;
    for (uint32_t i = 0; i < 256u; ++i) {
        const float b = __uint_as_float((uint32_t)(base + i));
        if (!__builtin_isfinite(b) || b == 0.0f) continue;
        m = fmax(m, __builtin_fabs(__builtin_fma(-(double)b, rcp64(b), 1.0)));
    }
    for (int o = 32; o > 0; o >>= 1) m = fmax(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63u) == 0u) atomicMax(out, (unsigned long long)__double_as_longlong(m));
}
__global__ __launch_bounds__(256) void selfcheck_sqrt_kernel(const float* x, float* y, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = sqrt_gate(x[i]);
}
}  // namespace

hipError_t selfcheck_rcp_error_host(double* max_err) {
    unsigned long long* d = nullptr;
    hipError_t e = hipMalloc(&d, sizeof *d);
    if (e == hipSuccess) e = hipMemset(d, 0, sizeof *d);
    if (e == hipSuccess) {
        // 65,536 workgroups x 256 threads x 256 patterns = 2^32
        hipLaunchKernelGGL(selfcheck_rcp_error_kernel, dim3(65536), dim3(256), 0, nullptr, d);
        e = hipGetLastError();
    }
    unsigned long long bits = 0;
    if (e == hipSuccess) e = hipMemcpy(&bits, d, sizeof bits, hipMemcpyDeviceToHost);
    if (d) hipFree(d);
    if (e == hipSuccess) std::memcpy(max_err, &bits, sizeof bits);
    return e;
}

hipError_t selfcheck_sqrt_host(const float* x, float* y, uint32_t n) {
    if (n == 0) return hipSuccess;
    const size_t bytes = (size_t)n * sizeof(float);
    float *dx = nullptr, *dy = nullptr;
    hipError_t e = hipMalloc(&dx, bytes);
    if (e == hipSuccess) e = hipMalloc(&dy, bytes);
    if (e == hipSuccess) e = hipMemcpy(dx, x, bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(selfcheck_sqrt_kernel, dim3((uint32_t)(((size_t)n + 255) / 256)), dim3(256), 0, nullptr, dx, dy, n);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(y, dy, bytes, hipMemcpyDeviceToHost);
    if (dx) hipFree(dx);
    if (dy) hipFree(dy);
    return e;
}

hipError_t selfcheck_divide_host(const float* a, const float* b, float* q, uint32_t n) {
    if (n == 0) return hipSuccess;
    const size_t bytes = (size_t)n * sizeof(float);
    float *da = nullptr, *db = nullptr, *dq = nullptr;
    hipError_t e = hipMalloc(&da, bytes);
    if (e == hipSuccess) e = hipMalloc(&db, bytes);
    if (e == hipSuccess) e = hipMalloc(&dq, bytes);
    if (e == hipSuccess) e = hipMemcpy(da, a, bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(db, b, bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(selfcheck_divide_kernel, dim3((uint32_t)(((size_t)n + 255) / 256)), dim3(256), 0, nullptr, da, db, dq, n);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(q, dq, bytes, hipMemcpyDeviceToHost);
    if (da) hipFree(da);
    if (db) hipFree(db);
    if (dq) hipFree(dq);
    return e;
}

hipError_t launch_detect_collisions(const ZenoAmdCollider* a, const ZenoAmdCollider* b, uint32_t n, ZenoAmdContactResult* out,
                                    hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const uint32_t blocks = (uint32_t)(((size_t)n + kCollideBlock - 1) / kCollideBlock);
    hipLaunchKernelGGL(detect_collisions_kernel, dim3(blocks), dim3(kCollideBlock), 0, stream, a, b, n, out);
    return hipGetLastError();
}

}  // namespace za
