// Attention at head sizes the MFMA kernels do not take: every multiple of 16 up to 112 other than 64 (16, 32, 48,
// 80, 96, 112), over the f16 and the int8 cache, computed in f32 on the vector ALUs. These are the reference's own
// f32 fallback kernels' cases: attention_partial (src/cuda.rs:1866-1932, and attention_partial_gqa's generic
// branch for a head size that is a multiple of 32, src/cuda.rs:1782-1864) for decode, and attention_prefill
// (src/cuda.rs:1934-2041) for prompts, which the reference runs for any head size up to 128 that its tensor-core
// kernels do not take (src/cuda.rs:8452-8476). Included by gi_attn_kernels.hip (one code object); the argument
// structs are that file's.
//
// Decode (gi_decode_f32 / _i8): one workgroup of 256 threads per (slice, head, token), over the slice's keys in
// tiles of 256: thread t scores key t of the tile (the dot product with Q * scale * log2(e), times the key's
// scale for int8), the workgroup takes the tile's max and an online base-2 softmax, and thread (g, d) adds
// p * V[key][d] over the keys g, g + 256/hd, ... of the tile (the value scale on p for int8). The slice's
// (unnormalised O, max, sum) go to the same partial rows gi_decode_combine merges; one slice writes the output.
// Prefill (gi_prefill_f32 / _i8): one workgroup of 256 threads per (head, 32 query rows); K and V tiles of 32 keys
// widened to f32 in LDS; thread (row r, lane c of 8) scores keys c, c + 8, c + 16, c + 24 of the tile for its row,
// and accumulates output dims c, c + 8, ... of that row.

#define F32_TILE 256 // decode: keys per tile (one per thread)
#define F32_MAXHD 128
#define PF32_ROWS 32 // prefill: query rows per workgroup
#define PF32_KT 32   // prefill: keys per tile

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

// 8 cache values from element offset `e` of a row: f16, or int8 (exact), as f32
template <bool I8>
__device__ __forceinline__ void gi_row8(const void* base, long long e, float (&x)[8]) {
    if constexpr (I8) {
        const u2 w = *reinterpret_cast<const u2*>(reinterpret_cast<const int8_t*>(base) + e);
#pragma unroll
        for (int i = 0; i < 8; i++) x[i] = (float)(int8_t)(((i < 4 ? w.x : w.y) >> (8 * (i & 3))) & 0xff);
    } else {
        const h8 h = __builtin_bit_cast(h8, *reinterpret_cast<const u4*>(reinterpret_cast<const uint16_t*>(base) + e));
#pragma unroll
        for (int i = 0; i < 8; i++) x[i] = (float)h[i];
    }
}
template <bool I8>
__device__ __forceinline__ float gi_elem(const void* base, long long e) {
    if constexpr (I8) return (float)reinterpret_cast<const int8_t*>(base)[e];
    else return (float)__builtin_bit_cast(_Float16, reinterpret_cast<const uint16_t*>(base)[e]);
}

template <bool I8>
__device__ __forceinline__ void gi_decode_f32_t(const GiDecodeArgs& a) {
    __shared__ float qs[F32_MAXHD];
    __shared__ float ps[F32_TILE];
    __shared__ float red[4];
    __shared__ float acc_sh[F32_TILE / 2][8]; // [key group][dim of the dim group] per dim group, see below
    const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
    const int hd = a.hd, G = a.n_heads / a.n_kv, kvh = h / G;
    const int pos0 = a.posp ? min(max(*a.posp, 0), a.kv_cap - a.n_tok) : a.pos0;
    const int kv_len = pos0 + a.n_tok;
    const int k_begin = s * a.chunk;
    const int nkeys = min(a.chunk, kv_len - k_begin);
    const int len = min(pos0 + b + 1 - k_begin, nkeys); // keys of the slice this token sees
    const long long kvs = a.kv_stride, khs = a.kv_head_stride;
    // P V: thread (key group g, dim group dg) takes 8 dims (one 16- or 8-byte load per key) of the keys g, g + groups,
    // ... of a tile; hd / 8 dim groups, groups = 256 / (hd / 8) key groups
    const int ndg = hd >> 3, groups = F32_TILE / ndg, g = tid / ndg, dg = tid % ndg;
    if (tid < hd) qs[tid] = a.q[(long long)b * a.q_stride + (long long)h * hd + tid] * a.qscale;
    __syncthreads();
    float m_run = GI_NEG_INF, l_run = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int t0 = 0; t0 < len; t0 += F32_TILE) {
        // scores of the tile: thread t, key t0 + t
        const int t = t0 + tid;
        float sc = GI_NEG_INF;
        if (t < len) {
            const long long row = (long long)(k_begin + t) * kvs + (long long)kvh * khs;
            float acc = 0.f;
            for (int e = 0; e < hd; e += 8) {
                float x[8];
                gi_row8<I8>(a.kc, row + e, x);
#pragma unroll
                for (int i = 0; i < 8; i++) acc = fmaf(qs[e + i], x[i], acc);
            }
            if constexpr (I8) acc *= a.ks[(long long)(k_begin + t) * a.sc_stride + (long long)kvh * a.sc_head_stride];
            sc = acc;
        }
        const float mx = gi_block_max(sc, red);
        const float m_new = fmaxf(m_run, mx); // key t0 of the tile is visible: finite
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        const float p = t < len ? __builtin_amdgcn_exp2f(sc - m_new) : 0.f;
        const float vsc = I8 && t < len ? a.vs[(long long)(k_begin + t) * a.sc_stride + (long long)kvh * a.sc_head_stride]
                                        : 1.f;
        ps[tid] = p * vsc; // the value scale rides on the weight, the sum is of the unscaled p
        const float psum = gi_block_sum(p, red); // (its barriers also publish ps)
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] *= alpha;
        if (g < groups) {
            const int kmax = min(F32_TILE, len - t0);
            for (int k = g; k < kmax; k += groups) {
                float x[8];
                gi_row8<I8>(a.vc, (long long)(k_begin + t0 + k) * kvs + (long long)kvh * khs + 8 * dg, x);
                const float pk = ps[k];
#pragma unroll
                for (int i = 0; i < 8; i++) o[i] = fmaf(pk, x[i], o[i]);
            }
        }
        __syncthreads(); // ps is rewritten by the next tile
    }
    // the key groups' sums, one dim group at a time through LDS (dim d = 8 dg + i)
    float O = 0.f;
    for (int dgi = 0; dgi < ndg; dgi++) {
        if (g < groups && dg == dgi) {
#pragma unroll
            for (int i = 0; i < 8; i++) acc_sh[g][i] = o[i];
        }
        __syncthreads();
        if (tid >= 8 * dgi && tid < 8 * dgi + 8)
            for (int k = 0; k < groups; k++) O += acc_sh[k][tid - 8 * dgi];
        __syncthreads();
    }
    if (tid < hd) {
        if (a.nsplit == 1) {
            a.out[(long long)b * a.out_stride + (long long)h * hd + tid] = len > 0 ? O / l_run : 0.f;
        } else {
            float* p = a.part + (((long long)b * a.n_heads + h) * a.nsplit + s) * (hd + 4);
            p[tid] = len > 0 ? O : 0.f;
            if (tid == 0) {
                p[hd] = len > 0 ? m_run : GI_NEG_INF;
                p[hd + 1] = len > 0 ? l_run : 0.f;
            }
        }
    }
}
extern "C" __global__ void __launch_bounds__(256) gi_decode_f32(GiDecodeArgs a) { gi_decode_f32_t<false>(a); }
extern "C" __global__ void __launch_bounds__(256) gi_decode_f32_i8(GiDecodeArgs a) { gi_decode_f32_t<true>(a); }

template <bool I8>
__device__ __forceinline__ void gi_prefill_f32_t(const GiPrefillArgs& a) {
    constexpr int LD = F32_MAXHD + 1; // padded rows: consecutive rows start in different banks
    __shared__ float Qs[PF32_ROWS][LD];
    __shared__ float Ks[PF32_KT][LD];
    __shared__ float Vs[PF32_KT][LD];
    __shared__ float Ps[PF32_ROWS][PF32_KT + 1];
    const int hd = a.hd, tid = threadIdx.x;
    const int G = a.n_heads / a.n_kv;
    const int qtiles = (a.n + PF32_ROWS - 1) / PF32_ROWS;
    const int h = blockIdx.x % a.n_heads, q0 = (qtiles - 1 - blockIdx.x / a.n_heads) * PF32_ROWS; // longest first
    const int kvh = h / G;
    const int r = tid >> 3, c = tid & 7; // this thread's row and lane
    const int kv_len = a.pos0 + a.n;
    const int kmax = min(kv_len, a.pos0 + q0 + PF32_ROWS);
    const long long kvs = a.kv_stride, khs = a.kv_head_stride;
    for (int i = tid; i < PF32_ROWS * hd; i += 256) {
        const int rr = i / hd, dd = i % hd, qr = min(q0 + rr, a.n - 1);
        const long long e = (long long)qr * a.q_stride + (long long)h * hd + dd;
        const float x = a.q_f16 ? (float)reinterpret_cast<const _Float16*>(a.q)[e] : reinterpret_cast<const float*>(a.q)[e];
        Qs[rr][dd] = x * a.qscale;
    }
    const int lim = a.pos0 + q0 + r; // the row's last visible key
    float m_run = GI_NEG_INF, l_run = 0.f, o[F32_MAXHD / 8];
#pragma unroll
    for (int i = 0; i < F32_MAXHD / 8; i++) o[i] = 0.f;
    for (int t0 = 0; t0 < kmax; t0 += PF32_KT) {
        __syncthreads(); // the previous tile is consumed (and Qs written, the first time)
        for (int i = tid; i < PF32_KT * hd; i += 256) {
            const int k = i / hd, dd = i % hd, kp = t0 + k;
            float kx = 0.f, vx = 0.f;
            if (kp < kv_len) {
                const long long e = (long long)kp * kvs + (long long)kvh * khs + dd;
                kx = gi_elem<I8>(a.kc, e);
                vx = gi_elem<I8>(a.vc, e);
                if constexpr (I8) {
                    const long long se = (long long)kp * a.sc_stride + (long long)kvh * a.sc_head_stride;
                    kx *= a.ks[se];
                    vx *= a.vs[se];
                }
            }
            Ks[k][dd] = kx;
            Vs[k][dd] = vx;
        }
        __syncthreads();
        float sc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int dd = 0; dd < hd; dd++) {
            const float q = Qs[r][dd];
#pragma unroll
            for (int j = 0; j < 4; j++) sc[j] = fmaf(q, Ks[c + 8 * j][dd], sc[j]);
        }
        float mx = GI_NEG_INF;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int kp = t0 + c + 8 * j;
            if (kp > lim || kp >= kv_len) sc[j] = GI_NEG_INF;
            mx = fmaxf(mx, sc[j]);
        }
        for (int m = 1; m < 8; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
        const float m_new = fmaxf(m_run, mx);
        // (a tile past the row's diagonal leaves the row as it is: every score is -inf and m_new may still be)
        const float alpha = m_new == GI_NEG_INF ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
        float ls = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float p = sc[j] == GI_NEG_INF ? 0.f : __builtin_amdgcn_exp2f(sc[j] - m_new);
            Ps[r][c + 8 * j] = p;
            ls += p;
        }
        for (int m = 1; m < 8; m <<= 1) ls += __shfl_xor(ls, m, 64);
        l_run = l_run * alpha + ls;
        m_run = m_new;
        // the row's 8 lanes are neighbours in one wave: their P writes are visible to each other after a wave barrier
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const int nd = hd >> 3;
#pragma unroll
        for (int i = 0; i < F32_MAXHD / 8; i++) {
            if (i < nd) {
                float acc = o[i] * alpha;
                for (int k = 0; k < PF32_KT; k++) acc = fmaf(Ps[r][k], Vs[k][c + 8 * i], acc);
                o[i] = acc;
            }
        }
    }
    const int qr = q0 + r;
    if (qr < a.n) {
        const float inv = 1.f / l_run;
        const int nd = hd >> 3;
#pragma unroll
        for (int i = 0; i < F32_MAXHD / 8; i++) {
            if (i < nd) {
                const long long e = (long long)qr * a.out_stride + (long long)h * hd + c + 8 * i;
                if (a.out_f16) reinterpret_cast<_Float16*>(a.out)[e] = (_Float16)(o[i] * inv);
                else reinterpret_cast<float*>(a.out)[e] = o[i] * inv;
            }
        }
    }
}
extern "C" __global__ void __launch_bounds__(256) gi_prefill_f32(GiPrefillArgs a) { gi_prefill_f32_t<false>(a); }
extern "C" __global__ void __launch_bounds__(256) gi_prefill_f32_i8(GiPrefillArgs a) { gi_prefill_f32_t<true>(a); }
