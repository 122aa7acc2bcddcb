// Peak probes for the measurement side (bench.py --workload peaks): what this box delivers, so that each
// kernel's roofline fraction can be read against the measured peaks as well as the published ones.
//  - gi_probe_mfma: v_mfma_f32_32x32x16_f16 only (the prefill's instruction), four independent accumulator
//    chains per wave, two waves per SIMD: the dense f16 MFMA rate at the clock the chip holds under it.
//  - gi_probe_read: a pure HBM read stream: each workgroup reads one contiguous chunk with 16 16-byte
//    loads in flight per lane, streaming (nt) cache policy (the decode's access pattern and policy).
// Not part of the attention path; built into their own code object, gi_probes_gfx950.hsaco.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// iters rounds of 32 MFMAs per wave (8 per chain); out receives one value per thread so that nothing is
// optimised away. flops per launch = gridDim.x * (blockDim.x / 64) * iters * 32 * 32768.
extern "C" __global__ void __launch_bounds__(256) gi_probe_mfma(int iters, float* out) {
    const int lane = threadIdx.x & 63;
    const h8 a = (h8)(_Float16)(lane * 1e-3f), b = (h8)(_Float16)(0.5f);
    f16x acc[4];
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[k][e] = 0.f;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int s = 0; s < 8; s++)
#pragma unroll
            for (int k = 0; k < 4; k++) acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[k], 0, 0, 0);
    }
    float r = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
        for (int e = 0; e < 16; e++) r += acc[k][e];
    out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

// Workgroup w reads 16-byte units [w * n16, (w + 1) * n16) of p; out gets a fold of the data (never equal to
// the sentinel in practice) so that the loads stay.
extern "C" __global__ void __launch_bounds__(256) gi_probe_read(const u4* __restrict__ p, long long n16, uint32_t* out) {
    constexpr int UNR = 16;
    const u4* b = p + (long long)blockIdx.x * n16;
    u4 acc = {0u, 0u, 0u, 0u};
    for (long long i = threadIdx.x; i < n16; i += 256 * UNR) {
        u4 v[UNR];
#pragma unroll
        for (int u = 0; u < UNR; u++) v[u] = i + u * 256 < n16 ? __builtin_nontemporal_load(b + i + u * 256) : u4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < UNR; u++) acc ^= v[u];
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) out[0] = 1u;
}
