/*
 * b3devcheck.hip - device evaluation of single math helpers of the engine.
 *
 * TEST INFRASTRUCTURE ONLY.  Runs the engine's own fd_atan2f, or_sinf and
 * or_cosf (puffysics_amd/csrc/b3d_math.h) on gfx950 over caller arrays, so
 * a GPU test can compare their bits with the host C library's.  Built with
 * the engine's flags (no contraction, no fast math, no packed fp32).
 */
#include <hip/hip_runtime.h>

#include "b3d_math.h"

__global__ void devcheck_atan2f_kernel(const float* y, const float* x, float* out, long n) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = b3d::fd_atan2f(y[i], x[i]);
}

extern "C" int devcheck_atan2f(const float* y, const float* x, float* out, long n, hipStream_t stream) {
    if (n <= 0) return 0;
    if (!y || !x || !out) return (int)hipErrorInvalidValue;
    long blocks = (n + 255) / 256;
    hipLaunchKernelGGL(devcheck_atan2f_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, y, x, out, n);
    return (int)hipGetLastError();
}

__global__ void devcheck_sincosf_kernel(const float* x, float* s, float* c, long n) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        s[i] = b3d::or_sinf(x[i]);
        c[i] = b3d::or_cosf(x[i]);
    }
}

extern "C" int devcheck_sincosf(const float* x, float* s, float* c, long n, hipStream_t stream) {
    if (n <= 0) return 0;
    if (!x || !s || !c) return (int)hipErrorInvalidValue;
    long blocks = (n + 255) / 256;
    hipLaunchKernelGGL(devcheck_sincosf_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, s, c, n);
    return (int)hipGetLastError();
}
