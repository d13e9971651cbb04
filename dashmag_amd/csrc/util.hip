// Small fill kernels used where a call must clear memory: kernels rather than hipMemsetAsync,
// so that a caller capturing the calls into a HIP graph records no memset nodes.
#include "attention_kernels.h"

namespace dm {

__global__ void fill_f32_kernel(float *p, float value, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = value;
}

__global__ void fill_zero_kernel(uint32_t *p, int64_t words, uint8_t *tail, int64_t tail_bytes) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (int64_t i = t; i < words; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0;
    if (t < tail_bytes) tail[t] = 0;
}

static unsigned grid_for(int64_t n) {
    int64_t g = (n + 255) / 256;
    if (g > 4096) g = 4096;
    return (unsigned)(g < 1 ? 1 : g);
}

void fill_f32(float *p, float value, int64_t n, hipStream_t st) {
    if (n <= 0) return;
    fill_f32_kernel<<<grid_for(n), 256, 0, st>>>(p, value, n);
}

void fill_zero(void *p, size_t bytes, hipStream_t st) {
    if (bytes == 0) return;
    // the buffers cleared here are 4-byte aligned allocations; odd tails are cleared bytewise
    int64_t words = (int64_t)(bytes / 4), tail = (int64_t)(bytes % 4);
    fill_zero_kernel<<<grid_for(words > tail ? words : tail), 256, 0, st>>>(
        (uint32_t *)p, words, (uint8_t *)p + words * 4, tail);
}

}  // namespace dm
