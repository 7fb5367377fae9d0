// stratametal_amd/csrc/smoe_synth.hip - seeded synthetic weights and activations for the benchmark
// configurations, generated on the device.  Same streams and arithmetic as the test oracle's generators
// (counter-based SplitMix64, Box-Muller with the library's own log and cos), so both fill bit-identical bytes.
#include "smoe_device.hpp"
#include "smoe_launch.hpp"

namespace smoe {

// Q2_0 block i: d = fp16(|sigma N(seed, 2s, i)|), code bytes from hash(seed, 2s+1, 2i) and (2i+1), little endian.
__global__ __launch_bounds__(256) void k_synth_q2_0(uint64_t seed, uint64_t st, int64_t nb, float sigma, uint8_t* out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nb) return;
    uint8_t* b = out + i * 18;
    const uint32_t d = f32_to_f16(__builtin_fabsf(sigma * normal_bm(seed, 2ull * st, (uint64_t)i)));
    b[0] = (uint8_t)d;
    b[1] = (uint8_t)(d >> 8);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint64_t v = hash64(seed, 2ull * st + 1ull, 2ull * (uint64_t)i + (uint64_t)h);
#pragma unroll
        for (int j = 0; j < 8; ++j) b[2 + 8 * h + j] = (uint8_t)(v >> (8 * j));
    }
}

// IQ2_S block i: d as above; the 80 other bytes from hash(seed, 2s+1, 10i + h), h < 10.
__global__ __launch_bounds__(256) void k_synth_iq2_s(uint64_t seed, uint64_t st, int64_t nb, float sigma, uint8_t* out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nb) return;
    uint8_t* b = out + i * 82;
    const uint32_t d = f32_to_f16(__builtin_fabsf(sigma * normal_bm(seed, 2ull * st, (uint64_t)i)));
    b[0] = (uint8_t)d;
    b[1] = (uint8_t)(d >> 8);
    for (int h = 0; h < 10; ++h) {
        const uint64_t v = hash64(seed, 2ull * st + 1ull, 10ull * (uint64_t)i + (uint64_t)h);
#pragma unroll
        for (int j = 0; j < 8; ++j) b[2 + 8 * h + j] = (uint8_t)(v >> (8 * j));
    }
}

__global__ __launch_bounds__(256) void k_synth_bf16(uint64_t seed, uint64_t st, int64_t n, float sigma, uint16_t* out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    out[i] = (uint16_t)f32_to_bf16(sigma * normal_bm(seed, st, (uint64_t)i));
}

__global__ __launch_bounds__(256) void k_synth_normal(uint64_t seed, uint64_t st, int64_t n, float sigma, float* out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    out[i] = sigma * normal_bm(seed, st, (uint64_t)i);
}

static dim3 grid_for(int64_t n) { return dim3((unsigned)((n + 255) / 256)); }

hipError_t launch_synth_blocks(int type, uint64_t seed, uint64_t st, int64_t nb, float sigma, uint8_t* out, hipStream_t s) {
    if (type == 22) hipLaunchKernelGGL(k_synth_iq2_s, grid_for(nb), dim3(256), 0, s, seed, st, nb, sigma, out);
    else hipLaunchKernelGGL(k_synth_q2_0, grid_for(nb), dim3(256), 0, s, seed, st, nb, sigma, out);
    return hipGetLastError();
}

hipError_t launch_synth_bf16(uint64_t seed, uint64_t st, int64_t n, float sigma, uint16_t* out, hipStream_t s) {
    hipLaunchKernelGGL(k_synth_bf16, grid_for(n), dim3(256), 0, s, seed, st, n, sigma, out);
    return hipGetLastError();
}

hipError_t launch_synth_normal(uint64_t seed, uint64_t st, int64_t n, float sigma, float* out, hipStream_t s) {
    hipLaunchKernelGGL(k_synth_normal, grid_for(n), dim3(256), 0, s, seed, st, n, sigma, out);
    return hipGetLastError();
}

}  // namespace smoe
