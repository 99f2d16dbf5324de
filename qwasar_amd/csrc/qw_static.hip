// qw_static.hip -- the device scratch of the allocation-free decode entry
// (qw_op_moe_layer_noalloc): one file-scope device array per GPU, sized at
// build time, which the library resolves once per device at init and never
// allocates or frees.
//
// The array's name is a host-side stand-in, not a device address, so host
// code never passes it to a kernel or a copy: qwk_static_init looks up its
// address on the current device with hipGetSymbolAddress, and every later
// use goes through that pointer (qwk_static_scratch).  Each GPU holds its own
// copy of the array at its own address, kept until the process ends.

#include <hip/hip_runtime.h>

#include "qw_kernels.h"

#define QWS_MAX_DEVICES 64

static __device__ __align__(256) unsigned char scratch[QWK_STATIC_SCRATCH_BYTES];

static void *qws_ptr[QWS_MAX_DEVICES];   // the array's address on each device, once resolved

// Zero fill with vector stores, one uint4 a thread (grid-stride).
__global__ void k_zero16(uint4 *p, size_t n16)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) p[i] = make_uint4(0, 0, 0, 0);
}

extern "C" int qwk_zero_fill(hipStream_t s, void *p, size_t bytes)
{
    if (bytes == 0) return 0;
    if (!p || ((uintptr_t)p & 15u) || (bytes & 15u)) return (int)hipErrorInvalidValue;
    const size_t n16 = bytes / 16;
    const unsigned blocks = (unsigned)(n16 / 256 + 1 < 1024 ? n16 / 256 + 1 : 1024);
    hipLaunchKernelGGL(k_zero16, dim3(blocks), dim3(256), 0, s, static_cast<uint4 *>(p), n16);
    return (int)hipGetLastError();
}

extern "C" int qwk_static_init(hipStream_t s)
{
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= QWS_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    if (qws_ptr[dev]) return 0;
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return (int)hipErrorInvalidSymbol;
    // a device global starts zeroed; cleared once more so that the contract
    // (the hand-off state at zero) does not rest on the loader
    const int rc = qwk_zero_fill(s, p, QWK_STATIC_SCRATCH_BYTES);
    if (rc != 0) return rc;
    e = hipStreamSynchronize(s);
    if (e != hipSuccess) return (int)e;
    qws_ptr[dev] = p;
    return 0;
}

extern "C" void *qwk_static_scratch(size_t *bytes)
{
    int dev = -1;
    if (bytes) *bytes = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= QWS_MAX_DEVICES || !qws_ptr[dev]) return nullptr;
    if (bytes) *bytes = QWK_STATIC_SCRATCH_BYTES;
    return qws_ptr[dev];
}
