// Peak probes for the measurement side (bench.py --workload peaks): what this box delivers, so that each
// kernel's roofline fraction can be read against the measured peaks as well as the published ones.
//  - gi_probe_mfma: v_mfma_f32_32x32x16_f16 only (the prefill's instruction), four independent accumulator
//    chains per wave, two waves per SIMD: the dense f16 MFMA rate at the clock the chip holds under it.
//  - gi_probe_mfma_rand: the same over pseudo-random operands that change every instruction (the power the
//    prefill's N(0,1) data draws, and so the clock the chip holds under it).
//  - gi_probe_read: a pure HBM read stream: each workgroup reads one contiguous chunk with 16 16-byte
//    loads in flight per lane, streaming (nt) cache policy (the decode's access pattern and policy).
//  - gi_probe_lds: LDS operand reads only, 16 in flight per lane, either ds_read_b128 (the prefill's K
//    fragments) or the transposing ds_read_b64_tr_b16 (its V^T fragments).
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

// The same instruction and schedule over operands that look like the prefill's: every lane holds 8 A and 8 B
// fragments of pseudo-random f16 values in [-2, 2) (a hash of lane and index), and consecutive MFMAs of a chain
// take different fragments, so the matrix core's inputs change every instruction as they do over N(0,1) K, Q,
// V and P. The dense rate then reflects the clock the chip holds under data that toggles (gi_probe_mfma's
// constant operands draw less power). flops per launch as gi_probe_mfma.
__device__ __forceinline__ h8 gi_probe_frag(uint32_t seed) {
    h8 r;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        uint32_t x = (seed * 8u + (uint32_t)e) * 2654435761u;
        x ^= x >> 15;
        x *= 2246822519u;
        x ^= x >> 13;
        r[e] = (_Float16)((float)(x >> 8) * (4.f / 16777216.f) - 2.f);
    }
    return r;
}
extern "C" __global__ void __launch_bounds__(256) gi_probe_mfma_rand(int iters, float* out) {
    const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    h8 a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a[i] = gi_probe_frag(g * 16u + (uint32_t)i);
        b[i] = gi_probe_frag(g * 16u + 8u + (uint32_t)i);
    }
    f16x acc[4];
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[k][e] = 0.f;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int s = 0; s < 8; s++)
#pragma unroll
            for (int k = 0; k < 4; k++)
                acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[(s + 2 * k) & 7], b[(s + 3 * k + 1) & 7], acc[k], 0, 0, 0);
    }
    float r = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
        for (int e = 0; e < 16; e++) r += acc[k][e];
    out[g] = r;
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

// LDS read rate: every lane issues `iters` rounds of 16 reads from a 32 KB LDS image, ds_read_b128 (tr = 0,
// 16 bytes per lane) or ds_read_b64_tr_b16 (tr = 1, 8 bytes per lane), conflict-free addresses; out gets a fold
// of the data (never equal to the sentinel in practice) so that the reads stay. Bytes per launch =
// gridDim.x * blockDim.x * iters * 16 * (tr ? 8 : 16).
typedef short gi_s4v __attribute__((__vector_size__(8)));
extern "C" __global__ void __launch_bounds__(256) gi_probe_lds(int iters, int tr, uint32_t* out) {
    __shared__ __attribute__((aligned(16))) uint32_t img[8192];
    for (int i = threadIdx.x; i < 8192; i += 256) img[i] = (uint32_t)i * 2654435761u;
    __syncthreads();
    const int lane = threadIdx.x & 63;
    uint32_t acc = 0u;
    if (tr) {
        const __attribute__((address_space(3))) unsigned short* base =
            (const __attribute__((address_space(3))) unsigned short*)(img);
        for (int it = 0; it < iters; it++) {
            gi_s4v v[16];
#pragma unroll
            for (int u = 0; u < 16; u++)
                v[u] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) gi_s4v*)(base + ((lane * 4 + u * 256 + (it & 1) * 128) & 16383)));
#pragma unroll
            for (int u = 0; u < 16; u++) acc ^= (uint32_t)(unsigned short)v[u][0] ^ ((uint32_t)(unsigned short)v[u][3] << 16);
            asm volatile("" ::: "memory");
        }
    } else {
        const __attribute__((address_space(3))) u4* base = (const __attribute__((address_space(3))) u4*)(img) + lane;
        for (int it = 0; it < iters; it++) {
            u4 v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = base[(u * 64 + (it & 1) * 32) & 2047];
#pragma unroll
            for (int u = 0; u < 16; u++) acc ^= v[u].x ^ v[u].w;
            asm volatile("" ::: "memory");
        }
    }
    if (acc == 0x9e3779b9u) out[0] = 1u;
}
