// Attention kernels for CDNA4 (gfx950): split-K flash decoding and causal flash prefill over a
// grouped-query f16 KV cache. Built offline into a code object (gi_attn_gfx950.hsaco) that the C-ABI
// library (gi_attn_host.cpp) loads with hipModuleLoad and launches by name.
//
// Cache layout (as the reference keeps it, src/cuda.rs:365-369, src/cuda.rs:10229-10242): K and V are
// separate buffers of rows [position][kv head][128] f16, kv_stride elements per position.
//
// Decode (reference semantics: attention_partial_gqa + attention_combine, src/cuda.rs:1684-1865,
// src/cuda.rs:2806-2836). One workgroup of 4 waves per (context slice, kv head, group of query
// (token, head) pairs). Each wave streams 32-key tiles of K and V straight from HBM into registers with
// 16-byte loads and runs both products on MFMA (v_mfma_f32_16x16x32_f16):
//   S^T[key, col] = K[key, :] . Qc[col, :]      col = (pair, hi|lo): Q*scale*log2(e) in f32 is split into
//                                               an f16 high part and an f16 remainder, so the two columns
//                                               of a pair sum to the f32 score (error ~2^-22 relative)
//   O^T[dim, col] += V^T[dim, key] . P^T[key, col]   col = (pair, hi|lo) of the f32 probability, same split
// Keys are ordered inside a tile so that the S^T accumulator a lane holds is exactly the B operand it
// needs for the PV product (no data movement between the two MFMAs); V is transposed 8x8 in registers.
// Online softmax is base 2 in f32. The 4 waves of a workgroup merge through LDS; the workgroup writes
// its slice's (unnormalised O, max, sum) or, with one slice, the normalised output. gi_decode_combine
// merges the slices.
//
// Prefill (reference semantics: attn_prefill_tc<128>, src/cuda.rs:2408-2617, without its rounding of
// Q*scale*log2(e) to f16: the scale is applied to the f32 scores). Defined further below.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

#define GI_NEG_INF (-__builtin_inff())
#define GI_LOG2E 1.4426950408889634f

// ------------------------------------------------------------------------------------------------ decode

// Arguments of the decode kernels (one struct so the host and the device agree on one definition).
struct GiDecodeArgs {
    const float* q;        // query rows: token b's head h at q + b*q_stride + h*128 (f32)
    const uint16_t* kc;    // K cache [pos][n_kv][128] f16, kv_stride elements per position
    const uint16_t* vc;    // V cache, same layout
    float* part;           // slice partials [token][head][nsplit][130]: O (128), max (base 2), sum
    float* out;            // output rows: token b's head h at out + b*out_stride + h*128 (f32)
    const int* posp;       // device position (overrides pos0 when non-null)
    long long q_stride;
    long long kv_stride;
    long long out_stride;
    int pos0;              // position of token 0: token b attends to keys 0..pos0+b
    int n_tok;
    int n_heads;
    int n_kv;
    int chunk;             // keys per slice, a multiple of 128
    int nsplit;            // slices per token (the grid's x)
    float qscale;          // scale * log2(e)
    int pad_;
};

#define DEC_WAVES 4
#define DEC_TILE 32
#define DEC_PAIRS 8 // (token, head) pairs per column block of 16 columns

__device__ __forceinline__ float wave_xor(float v, int m) { return __shfl_xor(v, m, 64); }

// Lane l of a wave: c = l % 16 (MFMA column / A-row), grp = l / 16 (k-group of 8).
template <int NCB>
__device__ __forceinline__ void gi_decode_partial_t(GiDecodeArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, grp = lane >> 4;
    const int s = blockIdx.x, kvh = blockIdx.y;
    const int pos0 = a.posp ? *a.posp : a.pos0;
    const int G = a.n_heads / a.n_kv;
    const int npairs = a.n_tok * G;
    const int pair0 = blockIdx.z * (DEC_PAIRS * NCB);
    const int kv_len = pos0 + a.n_tok; // keys any token of the launch may see
    const int k_begin = s * a.chunk;
    const int k_end = min(k_begin + a.chunk, kv_len);

    // this lane's column(s): pair and hi/lo half; span of the pair's token
    int span[NCB];
    bool valid[NCB];
    h8 qf[NCB][4]; // B operand of S^T = K Qc^T: k-step kk covers dims 32kk..32kk+31, this lane dims 32kk+8grp..+7
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
        int pi = pair0 + cb * DEC_PAIRS + (c >> 1);
        valid[cb] = pi < npairs;
        int t = valid[cb] ? pi / G : 0, g = valid[cb] ? pi % G : 0;
        span[cb] = valid[cb] ? pos0 + t + 1 : 0;
        const float* qrow = a.q + (long long)t * a.q_stride + (long long)(kvh * G + g) * 128;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const float4* qp = reinterpret_cast<const float4*>(qrow + 32 * kk + 8 * grp);
            float4 x0 = valid[cb] ? qp[0] : make_float4(0.f, 0.f, 0.f, 0.f);
            float4 x1 = valid[cb] ? qp[1] : make_float4(0.f, 0.f, 0.f, 0.f);
            float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float v = xs[e] * a.qscale;
                _Float16 hi = (_Float16)v;
                qf[cb][kk][e] = (c & 1) ? (_Float16)(v - (float)hi) : hi;
            }
        }
    }

    float m_run[NCB], l_run[NCB];
    f4 o[NCB][8]; // O^T: MFMA dd holds rows m = dims 8m + dd; this lane rows 4grp..4grp+3 -> dims 32grp + 8j + dd
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
        m_run[cb] = GI_NEG_INF;
        l_run[cb] = 0.f;
#pragma unroll
        for (int dd = 0; dd < 8; dd++) o[cb][dd] = f4{0.f, 0.f, 0.f, 0.f};
    }

    const long long kvs = a.kv_stride;
    const uint16_t* kbase = a.kc + (long long)kvh * 128;
    const uint16_t* vbase = a.vc + (long long)kvh * 128;
    // A-row r = c of S^T block b holds tile key 8*(c/4) + 4b + c%4; V: this lane loads keys 8grp+i, dims 8c..8c+7
    const int krow0 = 8 * (c >> 2) + (c & 3);

    for (int t0 = k_begin + wave * DEC_TILE; t0 < k_end; t0 += DEC_WAVES * DEC_TILE) {
        // ---- loads: K (2 blocks x 4 k-steps), V (8 keys), 16 bytes each; zeros past the keys in use
        u4 kw[2][4], vw[8];
#pragma unroll
        for (int b = 0; b < 2; b++) {
            int key = t0 + krow0 + 4 * b;
            const u4* kp = reinterpret_cast<const u4*>(kbase + (long long)key * kvs + 8 * grp);
#pragma unroll
            for (int kk = 0; kk < 4; kk++) kw[b][kk] = key < k_end ? kp[4 * kk] : u4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            int key = t0 + 8 * grp + i;
            vw[i] = key < k_end ? *reinterpret_cast<const u4*>(vbase + (long long)key * kvs + 8 * c) : u4{0u, 0u, 0u, 0u};
        }
        // ---- V^T: vt[dd] = the 8 keys' values of dim 8c + dd
        h8 vt[8];
#pragma unroll
        for (int dd = 0; dd < 8; dd++) {
            u4 w;
#pragma unroll
            for (int p = 0; p < 4; p++) {
                uint32_t lo = vw[2 * p][dd >> 1], hi = vw[2 * p + 1][dd >> 1];
                w[p] = (dd & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
            }
            vt[dd] = __builtin_bit_cast(h8, w);
        }
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
            // ---- S^T blocks: this lane gets column c, tile keys 8grp + 4b + j
            f4 sacc[2];
#pragma unroll
            for (int b = 0; b < 2; b++) {
                sacc[b] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < 4; kk++)
                    sacc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, kw[b][kk]), qf[cb][kk], sacc[b], 0, 0, 0);
            }
            float sc[8], mx = GI_NEG_INF;
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float v = sacc[b][j];
                    v = v + wave_xor(v, 1); // hi + lo columns of the pair (same sum in both lanes)
                    int key = t0 + 8 * grp + 4 * b + j;
                    v = key < span[cb] ? v : GI_NEG_INF;
                    sc[4 * b + j] = v;
                    mx = fmaxf(mx, v);
                }
            mx = fmaxf(mx, wave_xor(mx, 16));
            mx = fmaxf(mx, wave_xor(mx, 32));
            float m_new = fmaxf(m_run[cb], mx);
            float m_use = m_new == GI_NEG_INF ? 0.f : m_new; // nothing seen yet: keep everything at zero
            float alpha = exp2f(m_run[cb] - m_use);
            m_run[cb] = m_new;
            float psum = 0.f;
            h8 pf;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float p = exp2f(sc[i] - m_use);
                psum += p;
                _Float16 hi = (_Float16)p;
                pf[i] = (c & 1) ? (_Float16)(p - (float)hi) : hi;
            }
            l_run[cb] = l_run[cb] * alpha + psum;
#pragma unroll
            for (int dd = 0; dd < 8; dd++) {
                o[cb][dd] *= alpha;
                o[cb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vt[dd], pf, o[cb][dd], 0, 0, 0);
            }
        }
    }

    // ---- wave results: l over the 4 k-groups, O hi + lo columns
    __shared__ float sm_o[DEC_WAVES][DEC_PAIRS * NCB][128];
    __shared__ float sm_m[DEC_WAVES][DEC_PAIRS * NCB], sm_l[DEC_WAVES][DEC_PAIRS * NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
        float l = l_run[cb];
        l += wave_xor(l, 16);
        l += wave_xor(l, 32);
        int pl = cb * DEC_PAIRS + (c >> 1);
#pragma unroll
        for (int dd = 0; dd < 8; dd++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float v = o[cb][dd][j];
                v += wave_xor(v, 1);
                if ((c & 1) == 0) sm_o[wave][pl][32 * grp + 8 * j + dd] = v;
            }
        if (lane < 16 && (c & 1) == 0) {
            sm_m[wave][pl] = m_run[cb];
            sm_l[wave][pl] = l;
        }
    }
    __syncthreads();
    // ---- merge the waves: thread -> (pair, dim)
    for (int idx = threadIdx.x; idx < DEC_PAIRS * NCB * 128; idx += 256) {
        int pl = idx >> 7, d = idx & 127;
        int pi = pair0 + pl;
        if (pi >= npairs) continue;
        float M = GI_NEG_INF;
#pragma unroll
        for (int w = 0; w < DEC_WAVES; w++) M = fmaxf(M, sm_m[w][pl]);
        float L = 0.f, O = 0.f;
        if (M != GI_NEG_INF) {
#pragma unroll
            for (int w = 0; w < DEC_WAVES; w++) {
                float wt = exp2f(sm_m[w][pl] - M);
                L += wt * sm_l[w][pl];
                O += wt * sm_o[w][pl][d];
            }
        }
        int t = pi / G, h = kvh * G + pi % G;
        if (a.nsplit == 1) {
            a.out[(long long)t * a.out_stride + (long long)h * 128 + d] = O / L;
        } else {
            float* p = a.part + (((long long)t * a.n_heads + h) * a.nsplit + s) * 130;
            p[d] = O;
            if (d == 0) { p[128] = M; p[129] = L; }
        }
    }
}

extern "C" __global__ void __launch_bounds__(256) gi_decode_partial_1(GiDecodeArgs a) { gi_decode_partial_t<1>(a); }
extern "C" __global__ void __launch_bounds__(256) gi_decode_partial_2(GiDecodeArgs a) { gi_decode_partial_t<2>(a); }

// Merge the slices of each (token, head): M = max m_s, w_s = 2^(m_s - M), out = sum w_s O_s / sum w_s l_s
// (attention_combine's maths in base 2; empty slices carry m = -inf and weigh nothing). One workgroup of
// 128 threads per (head, token); thread d owns output dim d.
extern "C" __global__ void __launch_bounds__(128) gi_decode_combine(GiDecodeArgs a) {
    __shared__ float wsh[1024];
    __shared__ float red[2];
    const int h = blockIdx.x, t = blockIdx.y, d = threadIdx.x;
    const float* p = a.part + ((long long)t * a.n_heads + h) * a.nsplit * 130;
    float M = GI_NEG_INF;
    for (int s = d; s < a.nsplit; s += 128) M = fmaxf(M, p[s * 130 + 128]);
    // block max: 2 waves
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    if ((d & 63) == 0) red[d >> 6] = M;
    __syncthreads();
    M = fmaxf(red[0], red[1]);
    const bool held = a.nsplit <= 1024;
    if (held)
        for (int s = d; s < a.nsplit; s += 128) wsh[s] = M == GI_NEG_INF ? 0.f : exp2f(p[s * 130 + 128] - M);
    __syncthreads();
    float L = 0.f, O = 0.f;
    for (int s = 0; s < a.nsplit; s++) {
        float w = held ? wsh[s] : (M == GI_NEG_INF ? 0.f : exp2f(p[s * 130 + 128] - M));
        L += w * p[s * 130 + 129];
        O += w * p[s * 130 + d];
    }
    a.out[(long long)t * a.out_stride + (long long)h * 128 + d] = O / L;
}

// ------------------------------------------------------------------------------------------------ prefill

// Arguments of gi_prefill_fwd (must match gi_attn_host.cpp).
struct GiPrefillArgs {
    const void* q;         // query rows (f32 or f16): token i's head h at q + i*q_stride + h*128
    const uint16_t* kc;    // K cache [pos][n_kv][128] f16 holding keys 0..pos0+n-1
    const uint16_t* vc;    // V cache
    void* out;             // output rows (f32 or f16), out_stride elements apart
    long long q_stride;
    long long kv_stride;
    long long out_stride;
    int pos0;              // position of query 0 (keys before it are all visible: chunked prefill)
    int n;                 // query tokens
    int n_heads;
    int n_kv;
    float qscale;          // scale * log2(e), applied to the f32 scores
    int q_f16;
    int out_f16;
    int pad_;
};

#define PF_BQ 128          // query rows per workgroup (4 waves x 32)
#define PF_BK 64           // keys per tile
#define PF_KLD 136         // K tile row stride in f16 (272 bytes: rows 4 banks apart)
#define PF_VLD 72          // V^T tile row stride in f16 (144 bytes)
#define PF_KBUF (PF_BK * PF_KLD)
#define PF_VBUF (128 * PF_VLD)

// One workgroup = (head, 128 query rows); wave w owns rows 32w..32w+31 of the tile. Per 64-key tile:
//   S^T[key, q] = K[key, :] . Q[q, :]       v_mfma_f32_32x32x16_f16, K from LDS (A), Q in registers (B)
//   O^T[d, q]  += V^T[d, key] . P^T[key, q]  V^T from LDS (A), P^T straight from the S^T accumulators (B)
// A-row r of S^T block bb holds tile key 32bb + 16(i/2) + 8h + 4(i%2) + j for r = 8i + 4h + j, so the 16
// values a lane holds per block are exactly the keys its PV B operand needs (k-step 2bb + i/2, element
// 4(i%2) + j). K/V tiles are double-buffered in LDS with one barrier per tile; threads 0-127 stage K rows,
// threads 128-255 stage V as 8x8 blocks transposed in registers. Causal: a wave stops at its last row's
// position; only tiles crossing the diagonal are masked. Work order: the grid is remapped so that each of
// the 8 XCDs (blockIdx round-robin) walks a contiguous run of (kv head, query tile, head) items, longest
// query tiles first, so one kv head's K/V stays in one XCD's L2.
extern "C" __global__ void __launch_bounds__(256, 2) gi_prefill_fwd(GiPrefillArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 sk[2][PF_KBUF];
    __shared__ __attribute__((aligned(16))) _Float16 sv[2][PF_VBUF];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.n_heads / a.n_kv;
    const int qtiles = (a.n + PF_BQ - 1) / PF_BQ;
    const int nwg = gridDim.x;
    int j = blockIdx.x;
    if ((nwg & 7) == 0) j = (j & 7) * (nwg >> 3) + (j >> 3);
    const int kvh = j / (qtiles * G);
    const int rest = j % (qtiles * G);
    const int qt = qtiles - 1 - rest / G;
    const int h = kvh * G + rest % G;
    const int q0 = qt * PF_BQ;
    const int kv_len = a.pos0 + a.n;
    const int k_lim = min(kv_len, a.pos0 + q0 + PF_BQ); // keys any row of the tile may see
    const int ntiles = (k_lim + PF_BK - 1) / PF_BK;

    // ---- Q as B operands: lane (col = l%32, half = l/32), k-step ks: dims 16ks + 8*half .. +7
    const int qcol = lane & 31, half = lane >> 5;
    const int qrow = q0 + 32 * wave + qcol;      // this lane's query row
    const int qpos = a.pos0 + qrow;              // its position
    h8 qf[8];
    {
        const bool ok = qrow < a.n;
        if (a.q_f16) {
            const _Float16* qp = (const _Float16*)a.q + (long long)(ok ? qrow : 0) * a.q_stride + h * 128 + 8 * half;
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                u4 w = ok ? *reinterpret_cast<const u4*>(qp + 16 * ks) : u4{0u, 0u, 0u, 0u};
                qf[ks] = __builtin_bit_cast(h8, w);
            }
        } else {
            const float* qp = (const float*)a.q + (long long)(ok ? qrow : 0) * a.q_stride + h * 128 + 8 * half;
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                float4 x0 = ok ? *reinterpret_cast<const float4*>(qp + 16 * ks) : make_float4(0.f, 0.f, 0.f, 0.f);
                float4 x1 = ok ? *reinterpret_cast<const float4*>(qp + 16 * ks + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
                qf[ks] = h8{(_Float16)x0.x, (_Float16)x0.y, (_Float16)x0.z, (_Float16)x0.w,
                            (_Float16)x1.x, (_Float16)x1.y, (_Float16)x1.z, (_Float16)x1.w};
            }
        }
    }

    // ---- staging roles
    const bool stage_k = tid < 128;
    const int st = tid & 127;
    // K: chunk ids st + 128i -> key (id / 16), 16-byte column (id % 16)
    // V: thread -> dim group dg = st / 8 (dims 8dg..8dg+7), key group kg = st % 8 (keys 8kg..8kg+7)
    const int vdg = st >> 3, vkg = st & 7;
    const uint16_t* kbase = a.kc + (long long)kvh * 128;
    const uint16_t* vbase = a.vc + (long long)kvh * 128;
    u4 stg[8];
    auto load_tile = [&](int t0) {
        if (stage_k) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                int id = st + 128 * i, key = t0 + (id >> 4);
                stg[i] = key < kv_len ? *reinterpret_cast<const u4*>(kbase + (long long)key * a.kv_stride + 8 * (id & 15))
                                      : u4{0u, 0u, 0u, 0u};
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                int key = t0 + 8 * vkg + i;
                stg[i] = key < kv_len ? *reinterpret_cast<const u4*>(vbase + (long long)key * a.kv_stride + 8 * vdg)
                                      : u4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto store_tile = [&](int buf) {
        if (stage_k) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                int id = st + 128 * i;
                *reinterpret_cast<u4*>(&sk[buf][(id >> 4) * PF_KLD + 8 * (id & 15)]) = stg[i];
            }
        } else {
#pragma unroll
            for (int dd = 0; dd < 8; dd++) {
                u4 w;
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    uint32_t lo = stg[2 * p][dd >> 1], hi = stg[2 * p + 1][dd >> 1];
                    w[p] = (dd & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
                }
                *reinterpret_cast<u4*>(&sv[buf][(8 * vdg + dd) * PF_VLD + 8 * vkg]) = w;
            }
        }
    };

    // ---- per-lane state: O^T (4 dim blocks of 32), running max (raw score units), partial row sum
    f16x o[4];
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[db][e] = 0.f;
    float m_run = GI_NEG_INF, l_run = 0.f;
    const int wave_first = a.pos0 + q0 + 32 * wave;  // position of the wave's first row
    const int wave_last = wave_first + 31;
    // A-operand row of this lane in an S^T block: key offset within the block
    const int r = lane & 31;
    const int kperm = 16 * ((r >> 3) >> 1) + 8 * ((r >> 2) & 1) + 4 * ((r >> 3) & 1) + (r & 3);
    const int khalf = lane >> 5; // A k-group: dims 16ks + 8*khalf

    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int it = 0; it < ntiles; it++) {
        const int t0 = it * PF_BK, buf = it & 1;
        if (it + 1 < ntiles) load_tile(t0 + PF_BK);
        if (t0 <= wave_last) {
            const _Float16* K = sk[buf];
            const _Float16* V = sv[buf];
            f16x s[2];
#pragma unroll
            for (int bb = 0; bb < 2; bb++) {
#pragma unroll
                for (int e = 0; e < 16; e++) s[bb][e] = 0.f;
                const _Float16* krow = K + (32 * bb + kperm) * PF_KLD + 8 * khalf;
#pragma unroll
                for (int ks = 0; ks < 8; ks++) {
                    h8 kf = *reinterpret_cast<const h8*>(krow + 16 * ks);
                    s[bb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ks], s[bb], 0, 0, 0);
                }
            }
            // lane holds, for query qcol: block bb, element 4i + jj -> tile key 32bb + 16(i/2) + 8*half + 4(i%2) + jj
            const bool diag = t0 + PF_BK - 1 > wave_first || t0 + PF_BK > kv_len;
            float mx = GI_NEG_INF;
            if (diag) {
#pragma unroll
                for (int bb = 0; bb < 2; bb++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int jj = 0; jj < 4; jj++) {
                            int key = t0 + 32 * bb + 16 * (i >> 1) + 8 * half + 4 * (i & 1) + jj;
                            float v = s[bb][4 * i + jj];
                            v = (key > qpos || key >= kv_len) ? GI_NEG_INF : v;
                            s[bb][4 * i + jj] = v;
                            mx = fmaxf(mx, v);
                        }
            } else {
#pragma unroll
                for (int bb = 0; bb < 2; bb++)
#pragma unroll
                    for (int e = 0; e < 16; e++) mx = fmaxf(mx, s[bb][e]);
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(m_run, mx);
            const float m_use = m_new == GI_NEG_INF ? 0.f : m_new;
            const float alpha = exp2f((m_run - m_use) * a.qscale);
            m_run = m_new;
            const float mo = -m_use * a.qscale;
            float psum = 0.f;
            h8 pf[4]; // PV B operands, k-step ks = 2bb + i/2, element 4(i%2) + jj
#pragma unroll
            for (int bb = 0; bb < 2; bb++)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
                        float p = exp2f(fmaf(s[bb][4 * i + jj], a.qscale, mo));
                        psum += p;
                        pf[2 * bb + (i >> 1)][4 * (i & 1) + jj] = (_Float16)p;
                    }
            l_run = l_run * alpha + psum;
#pragma unroll
            for (int db = 0; db < 4; db++) {
                o[db] *= alpha;
                const _Float16* vrow = V + (32 * db + r) * PF_VLD + 8 * khalf;
#pragma unroll
                for (int ks = 0; ks < 4; ks++) {
                    h8 vf = *reinterpret_cast<const h8*>(vrow + 16 * ks);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[ks], o[db], 0, 0, 0);
                }
            }
        }
        if (it + 1 < ntiles) store_tile(buf ^ 1);
        __syncthreads();
    }

    // ---- normalise and write: lane holds query qcol, dims 32db + 8i + 4*half + jj
    float l = l_run + __shfl_xor(l_run, 32, 64);
    if (qrow < a.n) {
        const float inv = 1.f / l;
        if (a.out_f16) {
            _Float16* op = (_Float16*)a.out + (long long)qrow * a.out_stride + h * 128 + 4 * half;
#pragma unroll
            for (int db = 0; db < 4; db++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                    h4 v = h4{(_Float16)(o[db][4 * i] * inv), (_Float16)(o[db][4 * i + 1] * inv),
                              (_Float16)(o[db][4 * i + 2] * inv), (_Float16)(o[db][4 * i + 3] * inv)};
                    *reinterpret_cast<h4*>(op + 32 * db + 8 * i) = v;
                }
        } else {
            float* op = (float*)a.out + (long long)qrow * a.out_stride + h * 128 + 4 * half;
#pragma unroll
            for (int db = 0; db < 4; db++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    *reinterpret_cast<float4*>(op + 32 * db + 8 * i) =
                        make_float4(o[db][4 * i] * inv, o[db][4 * i + 1] * inv, o[db][4 * i + 2] * inv, o[db][4 * i + 3] * inv);
        }
    }
}
