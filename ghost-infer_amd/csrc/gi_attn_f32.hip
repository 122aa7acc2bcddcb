// Attention at head sizes the f16 MFMA kernels do not take: every multiple of 16 up to 112 other than 64 (16, 32, 48,
// 80, 96, 112), over the f16 and the int8 cache, computed in f32 with no f16 rounding of Q or P. These are the
// reference's own f32 fallback kernels' cases: attention_partial (src/cuda.rs:1866-1932, and attention_partial_gqa's
// generic branch for a head size that is a multiple of 32, src/cuda.rs:1782-1864) for decode, and attention_prefill
// (src/cuda.rs:1934-2041) for prompts, which the reference runs for any head size up to 128 that its tensor-core
// kernels do not take (src/cuda.rs:8452-8476). Included by gi_attn_kernels.hip (one code object); the argument
// structs are that file's. Each kernel is built per head size (gi_decode_f32_h80, gi_prefill_f32_i8_h96, ...), so
// every row loop is unrolled and a tile's loads all go out before their first use.
//
// Decode (gi_decode_f32_*): one workgroup of 256 threads per (slice, head, token), memory-bound. Per tile of 256
// keys every thread issues its loads at once: thread t the row of key t (its score), thread (g, dg) dims 8dg..8dg+7
// of the keys g, g + 256/(hd/8), ... (its share of P V). The score is the dot product with Q * scale * log2(e)
// (times the key's scale for int8); the workgroup takes the tile's max and an online base-2 softmax; the value
// scale rides on p. The slice's (unnormalised O, max, sum) go to the partial rows gi_decode_combine merges; one
// slice writes the output.
// Prefill (gi_prefill_f32_*): one workgroup of 8 waves per (head, 128 query rows), on v_mfma_f32_16x16x4f32 (f32
// operands, f32 accumulation). Tiles of 64 keys are widened to f32 in LDS (int8: times their scales) through
// registers, the next tile's loads in flight while the current one is used. A wave holds 16 query rows: S^T blocks
// (16 keys x 16 queries) from K (A) and Q^T (B, in registers); a lane then holds the scores of keys 4(l/16)..+3 of
// each block for query l%16, which is exactly the B operand of O^T = V^T P^T when k-step (block, r) takes the keys
// 4(l/16) + r of the block, so no score moves between lanes.

#define F32_TILE 256 // decode: keys per tile (one per thread)
#define PF32_WAVES 8
#define PF32_ROWS (16 * PF32_WAVES) // prefill: query rows per workgroup
#define PF32_KT 64                  // prefill: keys per tile

__device__ __forceinline__ float gi_block_max(float v, float* red) {
    for (int m = 32; m > 0; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
__device__ __forceinline__ float gi_block_sum(float v, float* red) {
    for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// 8 cache values of a row from element offset e: 16 bytes of f16, or 8 bytes of int8
template <bool I8> using GiRaw8 = typename gi_pick<I8, u2, u4>::type;
template <bool I8>
__device__ __forceinline__ GiRaw8<I8> gi_raw8(const void* base, long long e) {
    if constexpr (I8) return *reinterpret_cast<const u2*>(reinterpret_cast<const int8_t*>(base) + e);
    else return *reinterpret_cast<const u4*>(reinterpret_cast<const uint16_t*>(base) + e);
}
// ... widened to f32 (exact)
template <bool I8>
__device__ __forceinline__ void gi_widen8(const GiRaw8<I8>& w, float (&x)[8]) {
    if constexpr (I8) {
#pragma unroll
        for (int i = 0; i < 8; i++) x[i] = (float)(int8_t)(((i < 4 ? w.x : w.y) >> (8 * (i & 3))) & 0xff);
    } else {
        const h8 h = __builtin_bit_cast(h8, w);
#pragma unroll
        for (int i = 0; i < 8; i++) x[i] = (float)h[i];
    }
}

template <bool I8, int HD>
__device__ __forceinline__ void gi_decode_f32_t(const GiDecodeArgs& a) {
    constexpr int NDG = HD / 8;                    // 8-dim groups of a row
    constexpr int GROUPS = F32_TILE / NDG;         // key groups of P V (threads past GROUPS * NDG take none)
    constexpr int KPT = (F32_TILE + GROUPS - 1) / GROUPS; // keys of a tile per P V thread
    __shared__ float qs[HD];
    __shared__ float ps[F32_TILE];
    __shared__ float red[4];
    __shared__ float acc_sh[GROUPS][HD];
    const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
    const int G = a.n_heads / a.n_kv, kvh = h / G;
    const int pos0 = a.posp ? min(max(*a.posp, 0), a.kv_cap - a.n_tok) : a.pos0;
    const int k_begin = s * a.chunk;
    const int nkeys = min(a.chunk, pos0 + a.n_tok - k_begin);
    const int len = min(pos0 + b + 1 - k_begin, nkeys); // keys of the slice this token sees
    const long long kvs = a.kv_stride;
    const long long base = (long long)k_begin * kvs + (long long)kvh * a.kv_head_stride;
    const long long sbase = (long long)k_begin * a.sc_stride + (long long)kvh * a.sc_head_stride;
    const int g = tid / NDG, dg = tid % NDG;
    const bool pv = g < GROUPS;
    if (tid < HD) qs[tid] = a.q[(long long)b * a.q_stride + (long long)h * HD + tid] * a.qscale;
    __syncthreads();
    float m_run = GI_NEG_INF, l_run = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int t0 = 0; t0 < len; t0 += F32_TILE) {
        // every load of the tile first; past the span a thread reads the slice's last visible key (finite data)
        // and its weight is 0
        const int last = len - 1, t = t0 + tid;
        const int tk = min(t, last);
        GiRaw8<I8> kx[NDG], vx[KPT];
#pragma unroll
        for (int i = 0; i < NDG; i++) kx[i] = gi_raw8<I8>(a.kc, base + (long long)tk * kvs + 8 * i);
        if (pv) {
#pragma unroll
            for (int j = 0; j < KPT; j++)
                vx[j] = gi_raw8<I8>(a.vc, base + (long long)min(t0 + g + GROUPS * j, last) * kvs + 8 * dg);
        }
        float ksc = 1.f, vsc = 1.f;
        if constexpr (I8) {
            ksc = a.ks[sbase + (long long)tk * a.sc_stride];
            vsc = a.vs[sbase + (long long)tk * a.sc_stride];
        }
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < NDG; i++) {
            float x[8];
            gi_widen8<I8>(kx[i], x);
#pragma unroll
            for (int e = 0; e < 8; e++) acc = fmaf(qs[8 * i + e], x[e], acc);
        }
        const bool live = t < len;
        const float sc = live ? acc * ksc : GI_NEG_INF;
        const float mx = gi_block_max(sc, red);
        const float m_new = fmaxf(m_run, mx); // key t0 of the tile is visible: finite
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        const float p = live ? __builtin_amdgcn_exp2f(sc - m_new) : 0.f;
        ps[tid] = p * vsc; // the value scale rides on the weight, the sum is of the unscaled p
        const float psum = gi_block_sum(p, red); // (its barriers also publish ps)
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] *= alpha;
        if (pv) {
#pragma unroll
            for (int j = 0; j < KPT; j++) {
                const int k = g + GROUPS * j;
                if (GROUPS * (j + 1) <= F32_TILE || k < F32_TILE) {
                    float x[8];
                    gi_widen8<I8>(vx[j], x);
                    const float pk = ps[k];
#pragma unroll
                    for (int i = 0; i < 8; i++) o[i] = fmaf(pk, x[i], o[i]);
                }
            }
        }
        __syncthreads(); // ps is rewritten by the next tile
    }
    // the key groups' sums of each dim through LDS
    if (pv) {
#pragma unroll
        for (int i = 0; i < 8; i++) acc_sh[g][8 * dg + i] = o[i];
    }
    __syncthreads();
    if (tid < HD) {
        float O = 0.f;
        for (int k = 0; k < GROUPS; k++) O += acc_sh[k][tid];
        if (a.nsplit == 1) {
            a.out[(long long)b * a.out_stride + (long long)h * HD + tid] = len > 0 ? O / l_run : 0.f;
        } else {
            float* p = a.part + (((long long)b * a.n_heads + h) * a.nsplit + s) * (HD + 4);
            p[tid] = len > 0 ? O : 0.f;
            if (tid == 0) {
                p[HD] = len > 0 ? m_run : GI_NEG_INF;
                p[HD + 1] = len > 0 ? l_run : 0.f;
            }
        }
    }
}

template <bool I8, int HD>
__device__ __forceinline__ void gi_prefill_f32_t(const GiPrefillArgs& a) {
    constexpr int LD = HD + 4;            // floats per LDS row: 16-byte aligned, and conflict-free operand reads
    constexpr int NDG = HD / 8;           // 8-dim staging units of a row
    constexpr int NU = PF32_KT * NDG;     // staging units of a tile
    constexpr int NT = 64 * PF32_WAVES;
    constexpr int UPT = (NU + NT - 1) / NT;
    constexpr int DB = HD / 16;           // O^T blocks of 16 dims
    __shared__ __attribute__((aligned(16))) float Ks[PF32_KT * LD];
    __shared__ __attribute__((aligned(16))) float Vs[PF32_KT * LD];
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lc = l & 15, lg = l >> 4;
    const int G = a.n_heads / a.n_kv;
    const int qtiles = (a.n + PF32_ROWS - 1) / PF32_ROWS;
    const int h = blockIdx.x % a.n_heads, q0 = (qtiles - 1 - blockIdx.x / a.n_heads) * PF32_ROWS; // longest first
    const int kvh = h / G;
    const int kv_len = a.pos0 + a.n;
    const int kend = min(kv_len, a.pos0 + q0 + PF32_ROWS); // keys the workgroup's rows see
    const int wq0 = q0 + 16 * w;                            // the wave's first row
    const int wend = min(kv_len, a.pos0 + wq0 + 16);        // keys the wave's rows see
    const int qrow = wq0 + lc;                              // this lane's query row
    const int lim = a.pos0 + qrow;                          // its last visible key
    const long long kvs = a.kv_stride, kbase = (long long)kvh * a.kv_head_stride;
    const long long sbase = (long long)kvh * a.sc_head_stride;

    // Q^T, the B operand of S^T = K Q^T: k-step 4j + i takes dim 16j + 4(l/16) + i, so that the K operand of four
    // k-steps is one 16-byte LDS read
    float qv[HD / 4];
    {
        const long long e0 = (long long)min(qrow, a.n - 1) * a.q_stride + (long long)h * HD + 4 * lg;
#pragma unroll
        for (int j = 0; j < HD / 16; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const long long e = e0 + 16 * j + i;
                const float x = a.q_f16 ? (float)reinterpret_cast<const _Float16*>(a.q)[e]
                                        : reinterpret_cast<const float*>(a.q)[e];
                qv[4 * j + i] = x * a.qscale;
            }
    }

    // staging: unit u = tid + NT i of a tile is key u / NDG, dims 8 (u % NDG) ..; keys past the cache's span read
    // its last key (finite data, masked out of the scores, weight 0)
    GiRaw8<I8> kr[UPT], vr[UPT];
    float ksr[UPT], vsr[UPT];
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = tid + NT * i;
            if (NU % NT == 0 || u < NU) {
                const int kp = min(t0 + u / NDG, kv_len - 1);
                const long long e = (long long)kp * kvs + kbase + 8 * (u % NDG);
                kr[i] = gi_raw8<I8>(a.kc, e);
                vr[i] = gi_raw8<I8>(a.vc, e);
                if constexpr (I8) {
                    ksr[i] = a.ks[(long long)kp * a.sc_stride + sbase];
                    vsr[i] = a.vs[(long long)kp * a.sc_stride + sbase];
                }
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = tid + NT * i;
            if (NU % NT == 0 || u < NU) {
                float x[8], y[8];
                gi_widen8<I8>(kr[i], x);
                gi_widen8<I8>(vr[i], y);
                if constexpr (I8) {
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        x[e] *= ksr[i];
                        y[e] *= vsr[i];
                    }
                }
                const int off = (u / NDG) * LD + 8 * (u % NDG);
                *reinterpret_cast<f4*>(&Ks[off]) = f4{x[0], x[1], x[2], x[3]};
                *reinterpret_cast<f4*>(&Ks[off + 4]) = f4{x[4], x[5], x[6], x[7]};
                *reinterpret_cast<f4*>(&Vs[off]) = f4{y[0], y[1], y[2], y[3]};
                *reinterpret_cast<f4*>(&Vs[off + 4]) = f4{y[4], y[5], y[6], y[7]};
            }
        }
    };

    f4 o[DB];
#pragma unroll
    for (int d = 0; d < DB; d++) o[d] = f4{0.f, 0.f, 0.f, 0.f};
    float m_run = GI_NEG_INF, l_run = 0.f; // l_run: this lane's keys only, summed over the row's lanes at the end
    load_tile(0);
    for (int t0 = 0; t0 < kend; t0 += PF32_KT) {
        __syncthreads(); // every wave is done with the previous tile
        store_tile();
        if (t0 + PF32_KT < kend) load_tile(t0 + PF32_KT);
        __syncthreads();
        if (t0 >= wend) continue; // past every row of this wave (uniform)
        // S^T: 4 blocks of 16 keys x 16 queries
        f4 s[4];
#pragma unroll
        for (int kb = 0; kb < 4; kb++) s[kb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < HD / 16; j++)
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                const f4 kx = *reinterpret_cast<const f4*>(&Ks[(16 * kb + lc) * LD + 16 * j + 4 * lg]);
#pragma unroll
                for (int i = 0; i < 4; i++) s[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kx[i], qv[4 * j + i], s[kb], 0, 0, 0);
            }
        // lane l holds key t0 + 16 kb + 4(l/16) + r of query row qrow in s[kb][r]
        const bool edge = t0 + PF32_KT - 1 > a.pos0 + wq0 || t0 + PF32_KT > kv_len; // a mask reaches this tile
        float mx = GI_NEG_INF;
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int kp = t0 + 16 * kb + 4 * lg + r;
                if (edge && (kp > lim || kp >= kv_len)) s[kb][r] = GI_NEG_INF;
                mx = fmaxf(mx, s[kb][r]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run, mx); // key 0 is visible to every row, so finite from the first tile on
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        float ls = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                s[kb][r] = __builtin_amdgcn_exp2f(s[kb][r] - m_new);
                ls += s[kb][r];
            }
        l_run = l_run * alpha + ls;
        m_run = m_new;
#pragma unroll
        for (int d = 0; d < DB; d++) o[d] *= alpha;
        // O^T += V^T P^T: k-step (kb, r) takes the keys 16 kb + 4(l/16) + r
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int d = 0; d < DB; d++)
                    o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(Vs[(16 * kb + 4 * lg + r) * LD + 16 * d + lc], s[kb][r],
                                                                o[d], 0, 0, 0);
    }
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (qrow < a.n) {
        // lane l holds dims 16 d + 4(l/16) + i of query row qrow
        const float inv = 1.f / l_run;
        const long long e0 = (long long)qrow * a.out_stride + (long long)h * HD + 4 * lg;
#pragma unroll
        for (int d = 0; d < DB; d++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const long long e = e0 + 16 * d + i;
                if (a.out_f16) reinterpret_cast<_Float16*>(a.out)[e] = (_Float16)(o[d][i] * inv);
                else reinterpret_cast<float*>(a.out)[e] = o[d][i] * inv;
            }
    }
}

#define GI_F32_KERNELS(HD)                                                                                              \
    extern "C" __global__ void __launch_bounds__(256) gi_decode_f32_h##HD(GiDecodeArgs a) { gi_decode_f32_t<false, HD>(a); } \
    extern "C" __global__ void __launch_bounds__(256) gi_decode_f32_i8_h##HD(GiDecodeArgs a) { gi_decode_f32_t<true, HD>(a); } \
    extern "C" __global__ void __launch_bounds__(64 * PF32_WAVES) gi_prefill_f32_h##HD(GiPrefillArgs a) {               \
        gi_prefill_f32_t<false, HD>(a);                                                                                 \
    }                                                                                                                   \
    extern "C" __global__ void __launch_bounds__(64 * PF32_WAVES) gi_prefill_f32_i8_h##HD(GiPrefillArgs a) {            \
        gi_prefill_f32_t<true, HD>(a);                                                                                  \
    }
// head sizes 64 and 128: the prompt kernel only, for f32-precision prompts (the reference's attention_prefill with the
// tensor-core prefill off, GHOST_INFER_NO_TC_ATT; its decode at these sizes is the MFMA split path, f32-precise)
#define GI_F32_PREFILL_KERNELS(HD)                                                                                      \
    extern "C" __global__ void __launch_bounds__(64 * PF32_WAVES) gi_prefill_f32_h##HD(GiPrefillArgs a) {               \
        gi_prefill_f32_t<false, HD>(a);                                                                                 \
    }                                                                                                                   \
    extern "C" __global__ void __launch_bounds__(64 * PF32_WAVES) gi_prefill_f32_i8_h##HD(GiPrefillArgs a) {            \
        gi_prefill_f32_t<true, HD>(a);                                                                                  \
    }
GI_F32_PREFILL_KERNELS(64)
GI_F32_PREFILL_KERNELS(128)
GI_F32_KERNELS(16)
GI_F32_KERNELS(32)
GI_F32_KERNELS(48)
GI_F32_KERNELS(80)
GI_F32_KERNELS(96)
GI_F32_KERNELS(112)
