// Batched extended narrow phase (narrow_phase.detectCollision) on the GPU.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/zeno_amd_ext.h"

namespace za {

// One lane per pair: out[i] = detectCollision(a[i], b[i]) for i < n; device pointers.
hipError_t launch_detect_collisions(const ZenoAmdCollider* a, const ZenoAmdCollider* b, uint32_t n, ZenoAmdContactResult* out,
                                    hipStream_t stream);

// The same on host arrays with no device allocation: operands and results are staged in the
// library's static device array (at most ZENO_AMD_NOALLOC_MAX_PAIRS pairs, else
// hipErrorInvalidValue). Blocking; calls that overlap on one GPU race for the array.
hipError_t detect_collisions_host_noalloc(const ZenoAmdCollider* a, const ZenoAmdCollider* b, uint32_t n,
                                          ZenoAmdContactResult* out);

// q[i] = a[i] / b[i] through the step kernel's shared-reciprocal division (dmath.h rcp64 and
// qdivs) on host arrays: copies in, runs on the current device, copies back, waits.
hipError_t selfcheck_divide_host(const float* a, const float* b, float* q, uint32_t n);
hipError_t selfcheck_sqrt_host(const float* x, float* y, uint32_t n);
hipError_t selfcheck_rcp_error_host(double* max_err);

}  // namespace za
