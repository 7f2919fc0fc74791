// Streaming-read bandwidth probe for measure_bw.py (a measurement tool, not part of the GEMM
// library's C ABI): every lane reads 16-byte words of a buffer in a grid-stride loop and folds
// them with XOR; one word per workgroup is written so the loads cannot be removed.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256)
read_kernel(const u4* __restrict__ buf, size_t n16, uint32_t* __restrict__ sink) {
    u4 acc = u4{0u, 0u, 0u, 0u};
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {          // four independent loads in flight
        const u4 a = buf[i], b = buf[i + stride], c = buf[i + 2 * stride], d = buf[i + 3 * stride];
        acc ^= a ^ b ^ c ^ d;
    }
    for (; i < n16; i += stride) acc ^= buf[i];
    uint32_t v = acc.x ^ acc.y ^ acc.z ^ acc.w;
    for (int o = 32; o > 0; o >>= 1) v ^= __shfl_xor(v, o, 64);
    __shared__ uint32_t part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

}  // namespace

// Read `bytes` (a multiple of 16) from the 16-byte aligned device buffer `buf` with `blocks`
// workgroups of 256 threads; `sink` holds at least `blocks` uint32.  Asynchronous on `stream`.
extern "C" int w4a16_bw_read(const void* buf, size_t bytes, uint32_t* sink, int blocks, void* stream) {
    if (!buf || !sink || blocks < 1 || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(buf) % 16 != 0) return 1;
    hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<const u4*>(buf), bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : 3;
}
