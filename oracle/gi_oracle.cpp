// gi_oracle — CPU restatement of ghost-infer's attention, used ONLY as test infrastructure.
//
// This library is the checker for the HIP attention path and the timed CPU baseline in bench.py.
// Nothing in the product path (ghost-infer_amd/) links, loads or calls it; only tests/, the smoke
// check in __graft_entry__.py and bench.py's cpu_baseline leg do.
//
// Functions and the reference code they restate (paths relative to the reference repository):
//   gio_f16_to_f32 / gio_f32_to_f16   src/quant.rs:10-60  (IEEE binary16, round to nearest even)
//   gio_dot_f32                       src/quant.rs:758-768 (8 independent lanes, then the tail)
//   gio_att_chunk / gio_max_splits    src/cuda.rs:1642-1644, src/cuda.rs:8426-8444 (slice arithmetic)
//   gio_attention                     src/model.rs:1320-1409 (Model::attention: work units of
//                                     (token, kv head, slice), per-slice softmax, serial LSE merge)
//   gio_decode_gpu                    src/cuda.rs:1684-1865 + 2806-2836 (attention_partial_gqa with
//                                     an f16 cache, head size 128, then attention_combine)
//   gio_prefill_tc                    src/cuda.rs:2408-2617 (attn_prefill_tc<128>: Q*scale*log2e and
//                                     P rounded to f16, base-2 online softmax over 32-key tiles)
//   gio_qk_norm_rope                  src/cuda.rs:437-486 with the f16 kv_store (src/cuda.rs:312-362):
//                                     RMSNorm of q/k heads, RoPE, K/V rows into the f16 cache
//   gio_kv_quant_i8                   src/cuda.rs:333-339 (kv_store with KV8: row max / 127, rint)
//   gio_qk_norm_rope_i8               src/cuda.rs:437-486 storing with kv_quant_i8
//   gio_prefill_tc256                 gio_prefill_tc at head size 256 (attention_prefill_tc256, src/cuda.rs:2623)
//   gio_prefill_tc64 / _tc64_i8       gio_prefill_tc at head size 64 (attention_prefill_tc64, src/cuda.rs:2620), f16 / KV8
//   gio_prefill_tc_i8 / _tc256_i8     gio_prefill_tc (head size 128 / 256) over the KV8 cache (src/cuda.rs:2466-2498, 2548-2605:
//                                     integer keys, score times key scale, P V with f16(p * vs * 2^10))
//   gio_decode_gpu_i8                 gio_decode_gpu over the KV8 cache (src/cuda.rs:209-226, 1758-1760,
//                                     1821-1827: key scale on the score, value scale on the weight)
//   gio_decode_tc256_i8               src/cuda.rs:2625-2802 (attention_decode_tc256 over the KV8 cache: head
//                                     size 256, f16 Q, P = f16(p * vscale * 2^10), l of the unrounded p) + the
//                                     attention_combine merge
//   gio_kv4_fwht                      src/cuda.rs:242-256 (kv4_fwht; hadamard_rows, src/cuda.rs:4675-4693, with
//                                     block 256 is the same transform)
//   gio_kv4_quant / gio_kv4_dequant   src/cuda.rs:340-357 (kv_store with KV4) / 238-240 (kv4_pair)
//   gio_qk_norm_rope_q4               src/cuda.rs:437-486 with KV4 (q, k rotated after RoPE; v rotated in the store)
//   gio_decode_tc256_q4               attention_decode_tc256 with KV4 (src/cuda.rs:2681-2760) + attention_combine
//   gio_prefill_tc256_q4              attention_prefill_tc256 with KV4 (src/cuda.rs:2495-2514)
//
// How each is pinned (tests/test_oracle.py): the f16 conversion exhaustively against numpy's float16
// and against src/quant.rs:1160-1169's known values; the attention functions against an independent
// float64 brute-force softmax attention, closed forms (one position -> V0, zero keys -> mean of V,
// one dominant key -> its V row), invariance to the split count, causality and GQA group symmetry,
// and torch's scaled_dot_product_attention. gio_qk_norm_rope against closed forms: position 0 leaves a
// head unrotated, every rotation keeps each pair's length, a one-hot pair element lands on its partner
// with the float64 sine and cosine, unit weights give a unit-RMS head, and the cache holds numpy's f16
// rounding of the result.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <limits>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------- f16 <-> f32 (src/quant.rs:10-60)
float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ff;
    uint32_t bits;
    if (exp == 0 && mant == 0) {
        bits = sign;
    } else if (exp == 0) { // subnormal: shift the mantissa up until its leading one is the implicit bit
        int e = 127 - 15 + 1;
        uint32_t m = mant;
        while ((m & 0x400) == 0) { m <<= 1; e -= 1; }
        bits = sign | ((uint32_t)e << 23) | ((m & 0x3ff) << 13);
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t f32_to_f16(float f) {
    uint32_t bits;
    std::memcpy(&bits, &f, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
    int exp = (int)((bits >> 23) & 0xff);
    uint32_t mant = bits & 0x7fffff;
    if (exp == 0xff) return sign | 0x7c00 | (mant ? 0x200 : 0);
    int e = exp - 127 + 15;
    if (e >= 0x1f) return sign | 0x7c00;
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = mant | 0x800000;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half = 1u << (shift - 1);
        uint32_t r = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        if (rem > half || (rem == half && (r & 1))) r += 1;
        return sign | (uint16_t)r;
    }
    uint32_t r = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (r & 1))) r += 1; // may carry into the exponent: still RNE
    return sign | (uint16_t)r;
}

// 65536-entry widening table: the f16 cache widened exactly to f32, row by row as it is read
struct WidenTable {
    float v[65536];
    WidenTable() { for (uint32_t i = 0; i < 65536; i++) v[i] = f16_to_f32((uint16_t)i); }
};
const WidenTable& widen() { static WidenTable t; return t; }

// ---------------------------------------------------------------- dot_f32 (src/quant.rs:758-768)
float dot_f32(const float* a, const float* b, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int full = n / 8 * 8;
    float tail = 0.f;
    for (int i = full; i < n; i++) tail += a[i] * b[i];
    for (int c = 0; c < full; c += 8)
        for (int i = 0; i < 8; i++) acc[i] += a[c + i] * b[c + i];
    float s = 0.f;
    for (int i = 0; i < 8; i++) s += acc[i];
    return s + tail;
}

// A cache row reader: f32 rows, or f16 rows widened into a scratch row.
struct Cache {
    const float* f32 = nullptr;
    const uint16_t* f16 = nullptr;
    long stride = 0; // elements per position
    const float* row(long t, int off, int len, float* tmp) const {
        if (f32) return f32 + t * stride + off;
        const uint16_t* p = f16 + t * stride + off;
        const float* w = widen().v;
        for (int i = 0; i < len; i++) tmp[i] = w[p[i]];
        return tmp;
    }
};

// Runs f(i) for i in [0, count) over `threads` workers (rayon's par_chunks_mut.for_each_init stand-in:
// every unit's arithmetic is independent of which worker runs it, so the results do not depend on it).
template <class F>
void parallel_for(long count, int threads, F f) {
    if (threads <= 1 || count <= 1) {
        for (long i = 0; i < count; i++) f(i);
        return;
    }
    std::atomic<long> next{0};
    std::vector<std::thread> pool;
    int nt = (int)std::min<long>(threads, count);
    for (int w = 0; w < nt; w++)
        pool.emplace_back([&] {
            for (long i; (i = next.fetch_add(1)) < count;) f(i);
        });
    for (auto& t : pool) t.join();
}

// ---------------------------------------------------------------- Model::attention (src/model.rs:1320-1409)
void model_attention(const float* q, long q_stride, const Cache& kc, const Cache& vc, float* out, long out_stride,
                     int pos0, int n, int n_heads, int n_kv, int hd, float scale, int threads) {
    const int group = n_heads / n_kv;
    const int kd = hd, vd = hd;
    auto span_of = [&](int b) { return pos0 + b + 1; }; // causal: token b sees positions 0..=pos0+b
    const long pairs = (long)n * n_kv;
    long splits;
    if (pairs >= threads) {
        splits = 1;
    } else {
        long a = (threads + pairs - 1) / pairs;
        long c = ((long)span_of(0) + 63) / 64;
        splits = std::max<long>(1, std::min(a, c));
    }
    const long unit = (long)group * vd + 2 * group; // per slice: unnormalised outputs, then (max, sum) per head
    std::vector<float> partial((size_t)(pairs * splits * unit), 0.f);

    auto slice_task = [&](long idx) {
        std::vector<float> scores, krow(kd), vrow(vd);
        float* part = partial.data() + idx * unit;
        long pair = idx / splits, split = idx % splits;
        int b = (int)(pair / n_kv), kvh = (int)(pair % n_kv);
        long span = span_of(b);
        long per = (span + splits - 1) / splits;
        long t0 = std::min(split * per, span), t1 = std::min((split + 1) * per, span);
        long len = t1 - t0;
        const float* qs = q + (long)b * q_stride + (long)kvh * group * kd;
        float* o = part;
        float* stats = part + (long)group * vd;
        std::fill(o, o + (long)group * vd, 0.f);
        if (len == 0) {
            for (int g = 0; g < group; g++) {
                stats[2 * g] = -std::numeric_limits<float>::infinity();
                stats[2 * g + 1] = 0.f;
            }
            return;
        }
        scores.assign((size_t)(group * len), 0.f);
        for (long t = t0; t < t1; t++) {
            const float* kt = kc.row(t, kvh * kd, kd, krow.data());
            for (int g = 0; g < group; g++) scores[g * len + (t - t0)] = dot_f32(qs + (long)g * kd, kt, kd) * scale;
        }
        for (int g = 0; g < group; g++) {
            float* row = scores.data() + g * len;
            float mx = -std::numeric_limits<float>::infinity();
            for (long i = 0; i < len; i++) mx = std::max(mx, row[i]);
            float total = 0.f;
            for (long i = 0; i < len; i++) {
                row[i] = std::exp(row[i] - mx);
                total += row[i];
            }
            stats[2 * g] = mx;
            stats[2 * g + 1] = total;
        }
        for (long t = t0; t < t1; t++) {
            const float* vt = vc.row(t, kvh * vd, vd, vrow.data());
            for (int g = 0; g < group; g++) {
                float w = scores[g * len + (t - t0)];
                float* oh = o + (long)g * vd;
                for (int d = 0; d < vd; d++) oh[d] += w * vt[d];
            }
        }
    };
    // a single token over a short context is too little work to be worth waking threads
    long work = (long)n * n_heads * (pos0 + n) * kd;
    parallel_for(pairs * splits, work < (1L << 16) ? 1 : threads, slice_task);

    // merge the slices of each (token, kv head) into normalised head outputs (serial, slice order)
    for (long pair = 0; pair < pairs; pair++) {
        int b = (int)(pair / n_kv), kvh = (int)(pair % n_kv);
        const float* parts = partial.data() + pair * splits * unit;
        for (int g = 0; g < group; g++) {
            float m = -std::numeric_limits<float>::infinity();
            for (long s = 0; s < splits; s++) m = std::max(m, parts[s * unit + (long)group * vd + 2 * g]);
            float* o = out + (long)b * out_stride + (long)(kvh * group + g) * vd;
            std::fill(o, o + vd, 0.f);
            float total = 0.f;
            for (long s = 0; s < splits; s++) {
                const float* p = parts + s * unit;
                float w = std::exp(p[(long)group * vd + 2 * g] - m);
                if (w == 0.f) continue;
                total += p[(long)group * vd + 2 * g + 1] * w;
                for (int d = 0; d < vd; d++) o[d] += w * p[(long)g * vd + d];
            }
            float inv = 1.f / total;
            for (int d = 0; d < vd; d++) o[d] *= inv;
        }
    }
}

// ---------------------------------------------------------------- slice arithmetic (src/cuda.rs:1642, 8426-8444)
constexpr int ATT_MAX_CHUNK = 256;
constexpr int SPLIT_MIN_SPAN = 32;
constexpr int ATT_TARGET_BLOCKS = 96;
int att_chunk(int span, int want, int cap) {
    if (span <= SPLIT_MIN_SPAN) return ATT_MAX_CHUNK;
    return std::min(std::max((span + want - 1) / want, 32), cap);
}

// ---------------------------------------------------------------- attention_partial_gqa + attention_combine
// (src/cuda.rs:1684-1865, 2806-2836), f16 cache, head size 128, restated for one block at a time.
float lane_dot(const float* q, const float* k) { // src/cuda.rs:1647-1649: fma chain over 4 products
    return std::fma(q[3], k[3], std::fma(q[2], k[2], std::fma(q[1], k[1], q[0] * k[0])));
}
// score of one key row for one head, in the butterfly order of src/cuda.rs:1716-1754
float butterfly_score(const float* qs, const float* k) {
    float s1[16];
    for (int j = 0; j < 16; j++) s1[j] = lane_dot(qs + 4 * j, k + 4 * j) + lane_dot(qs + 4 * j + 64, k + 4 * j + 64);
    float s2[8], s3[4], s4[2];
    for (int j = 0; j < 8; j++) s2[j] = s1[j] + s1[j + 8];
    for (int j = 0; j < 4; j++) s3[j] = s2[j] + s2[j + 4];
    for (int j = 0; j < 2; j++) s4[j] = s3[j] + s3[j + 2];
    return s4[0] + s4[1];
}
// block_sum over 128 threads (src/cuda.rs:148-168): per-thread strided sums, warp_sum by shfl_down, then
// warp 0 sums the 4 warp totals the same way
float block_sum128(const float* per_thread) {
    float w[4];
    for (int wp = 0; wp < 4; wp++) {
        float v[32];
        for (int l = 0; l < 32; l++) v[l] = per_thread[32 * wp + l];
        for (int o = 16; o > 0; o >>= 1)
            for (int l = 0; l < 32; l++) if (l + o < 32) v[l] = v[l] + v[l + o];
        w[wp] = v[0];
    }
    float v[32] = {0};
    for (int i = 0; i < 4; i++) v[i] = w[i];
    for (int o = 16; o > 0; o >>= 1)
        for (int l = 0; l < 32; l++) if (l + o < 32) v[l] = v[l] + v[l + o];
    return v[0];
}

void combine(const float* part_base, float* out, long out_stride, int pos0, int m, int n_heads, int hd, int nsplit,
             int want, int cap);

// A cache element as the kernels widen it: f16 bits exactly, int8 as its integer value.
inline float kv_value(uint16_t h) { return widen().v[h]; }
inline float kv_value(int8_t v) { return (float)v; }

// KV_T = uint16_t: the f16 cache (scales are 1: KV_SCALE's products are exact). KV_T = int8_t: the KV8 cache
// (src/cuda.rs:209-226) with f32 scales ks / vs [pos][n_kv]: score = butterfly dot * key scale (src/cuda.rs:1758-
// 1760), the value scale rides on the weight and the exp-sum is of the unscaled exponentials (src/cuda.rs:1821-
// 1827).
template <typename KV_T>
void decode_gpu(const float* qkv, long q_stride, const KV_T* kc, const KV_T* vc, const float* ks, const float* vs,
                long kv_stride, float* out, long out_stride, int pos0, int m, int n_heads, int n_kv, float scale,
                int nsplit, int want, int cap, int threads) {
    const int hd = 128, G = n_heads / n_kv;
    // partials [token][head][slice][hd + 2]: (unnormalised O, max, exp-sum) in natural-log units
    std::vector<float> part((size_t)m * n_heads * nsplit * (hd + 2), 0.f);
    auto block = [&](long idx) { // one block = (kv head, token, slice)
        int s = (int)(idx % nsplit);
        int b = (int)((idx / nsplit) % m);
        int kvh = (int)(idx / nsplit / m);
        int span = pos0 + b + 1;
        int chunk = att_chunk(span, want, cap);
        int t0 = s * chunk, len = std::min(span, t0 + chunk) - t0;
        auto P = [&](int g) { return part.data() + (((size_t)b * n_heads + kvh * G + g) * nsplit + s) * (hd + 2); };
        if (len <= 0) {
            for (int g = 0; g < G; g++) {
                float* p = P(g);
                std::fill(p, p + hd, 0.f);
                p[hd] = -std::numeric_limits<float>::infinity();
                p[hd + 1] = 0.f;
            }
            return;
        }
        std::vector<float> qsh((size_t)G * hd), sc((size_t)len * G), krow(hd);
        const float* qb = qkv + (long)b * q_stride + (long)kvh * G * hd;
        for (int i = 0; i < G * hd; i++) qsh[i] = qb[i] * scale;
        for (int t = 0; t < len; t++) {
            const KV_T* kt = kc + (long)(t0 + t) * kv_stride + kvh * hd;
            for (int i = 0; i < hd; i++) krow[i] = kv_value(kt[i]);
            const float kscale = ks ? ks[(long)(t0 + t) * n_kv + kvh] : 1.f;
            for (int g = 0; g < G; g++)
                sc[(size_t)t * G + g] = butterfly_score(qsh.data() + g * hd, krow.data()) * kscale;
        }
        for (int g = 0; g < G; g++) {
            float mx = -std::numeric_limits<float>::infinity();
            for (int t = 0; t < len; t++) mx = std::max(mx, sc[(size_t)t * G + g]);
            float thr[128] = {0};
            for (int t = 0; t < len; t++) {
                float e = std::exp(sc[(size_t)t * G + g] - mx);
                sc[(size_t)t * G + g] = e * (vs ? vs[(long)(t0 + t) * n_kv + kvh] : 1.f);
                thr[t % 128] = thr[t % 128] + e;
            }
            float seg = block_sum128(thr);
            for (int d = 0; d < hd; d++) {
                float a = 0.f;
                for (int t = 0; t < len; t++)
                    a = std::fma(sc[(size_t)t * G + g], kv_value(vc[(long)(t0 + t) * kv_stride + kvh * hd + d]), a);
                int h = kvh * G + g;
                if (nsplit == 1) {
                    out[(long)b * out_stride + (long)h * hd + d] = a * (1.f / seg);
                } else {
                    float* p = P(g);
                    p[d] = a;
                    if (d == 0) { p[hd] = mx; p[hd + 1] = seg; }
                }
            }
        }
    };
    parallel_for((long)n_kv * m * nsplit, threads, block);
    if (nsplit > 1) combine(part.data(), out, out_stride, pos0, m, n_heads, hd, nsplit, want, cap);
}

// attention_combine (src/cuda.rs:2806-2836): per (token, head) the slices' max, each slice's weight exp(m_s -
// max), the weighted exp-sums and outputs in slice order. part: [token][head][slice][hd + 2], natural log.
void combine(const float* part_base, float* out, long out_stride, int pos0, int m, int n_heads, int hd, int nsplit,
             int want, int cap) {
    for (int b = 0; b < m; b++)
        for (int h = 0; h < n_heads; h++) {
            int span = pos0 + b + 1;
            int chunk = att_chunk(span, want, cap);
            int used = std::min(nsplit, (span + chunk - 1) / chunk);
            const float* p = part_base + ((size_t)b * n_heads + h) * nsplit * (hd + 2);
            float mm = -std::numeric_limits<float>::infinity();
            for (int s = 0; s < used; s++) mm = std::max(mm, p[s * (hd + 2) + hd]);
            std::vector<float> w(used);
            for (int s = 0; s < used; s++) w[s] = std::exp(p[s * (hd + 2) + hd] - mm);
            float total = 0.f;
            for (int s = 0; s < used; s++) total = std::fma(p[s * (hd + 2) + hd + 1], w[s], total);
            float inv = 1.f / total;
            for (int d = 0; d < hd; d++) {
                float acc = 0.f;
                for (int s = 0; s < used; s++) acc = std::fma(p[s * (hd + 2) + d], w[s], acc);
                out[(long)b * out_stride + (long)h * hd + d] = acc * inv;
            }
        }
}

// ---------------------------------------------------------------- attention_decode_tc256, KV8 (src/cuda.rs:2625-2802)
// The tensor-core decode of 256-wide grouped heads over the int8 cache, on attention_partial_gqa's grid and
// slices (its partials merged by attention_combine). Per block (kv head, token, slice), warp w of 4 takes the
// slice's 8-position tiles w, w + 4, ...: Q rounded to f16 after scaling by scale*log2(e); per tile the scores
// (the f16 Q times the integer keys, f32 sums) times the key scales; the running max moves every tile
// (alpha = exp2(m - m_new)); l = alpha*l + the unrounded p; P = f16(p * vscale * 2^10) and O = alpha*O + P V.
// Warps 1..3 merge into warp 0 in order; out = O / 2^10 / l, or the partial (O / 2^10, m*ln2, l).
// KV_T = uint16_t (the KV4 build, src/cuda.rs:2681-2700, 2725-2760): the fragments are the f16 values
// f16((n - 8) * scale) of the 4-bit cache (dequantised beforehand) and the key / value scale factors are 1
// (KV_SCALE, src/cuda.rs:233), so ks / vs are null: scores are the plain dot products, P = f16(p * 2^10).
template <typename KV_T>
void decode_tc256(const float* qkv, long q_stride, const KV_T* kc, const KV_T* vc, const float* ks,
                  const float* vs, long kv_stride, float* out, long out_stride, int pos0, int m, int n_heads, int n_kv,
                  float scale, int nsplit, int want, int cap, int threads) {
    const int hd = 256, G = n_heads / n_kv;
    const float NEG = -std::numeric_limits<float>::infinity(), LN2 = 0.6931471805599453f, BIAS = 1024.f;
    const float qs = scale * 1.4426950408889634f;
    std::vector<float> part((size_t)m * n_heads * nsplit * (hd + 2), 0.f);
    auto block = [&](long idx) {
        int s = (int)(idx % nsplit);
        int b = (int)((idx / nsplit) % m);
        int kvh = (int)(idx / nsplit / m);
        int span = pos0 + b + 1;
        int chunk = att_chunk(span, want, cap);
        int t0 = s * chunk, len = std::min(span, t0 + chunk) - t0;
        auto P = [&](int g) { return part.data() + (((size_t)b * n_heads + kvh * G + g) * nsplit + s) * (hd + 2); };
        if (len <= 0) {
            for (int g = 0; g < G; g++) {
                float* p = P(g);
                std::fill(p, p + hd, 0.f);
                p[hd] = NEG;
                p[hd + 1] = 0.f;
            }
            return;
        }
        // Q as the f16 fragments hold it
        std::vector<float> qh((size_t)G * hd);
        const float* qb = qkv + (long)b * q_stride + (long)kvh * G * hd;
        for (int i = 0; i < G * hd; i++) qh[i] = f16_to_f32(f32_to_f16(qb[i] * qs));
        // per warp and head: running max, sum, O
        std::vector<float> wm(4 * G, NEG), wl(4 * G, 0.f), wo((size_t)4 * G * hd, 0.f);
        for (int w = 0; w < 4; w++)
            for (int tt = 8 * w; tt < len; tt += 32)
                for (int g = 0; g < G; g++) {
                    float sc[8], mx = NEG;
                    for (int j = 0; j < 8; j++) {
                        int pa = tt + j;
                        if (pa >= len) { sc[j] = NEG; continue; }
                        const KV_T* kr = kc + (long)(t0 + pa) * kv_stride + kvh * hd;
                        float acc = 0.f;
                        for (int d = 0; d < hd; d++) acc += qh[(size_t)g * hd + d] * kv_value(kr[d]);
                        sc[j] = ks ? acc * ks[(long)(t0 + pa) * n_kv + kvh] : acc;
                        mx = std::max(mx, sc[j]);
                    }
                    float& mr = wm[w * G + g];
                    float& lr = wl[w * G + g];
                    float* o = wo.data() + ((size_t)w * G + g) * hd;
                    const float mn = std::max(mr, mx), alpha = std::exp2(mr - mn);
                    mr = mn;
                    float psum = 0.f, pv[8];
                    for (int j = 0; j < 8; j++) {
                        const float p = std::exp2(sc[j] - mn);
                        psum += p;
                        const float v = tt + j < len ? (vs ? vs[(long)(t0 + tt + j) * n_kv + kvh] : 1.f) * BIAS : 0.f;
                        pv[j] = f16_to_f32(f32_to_f16(p * v));
                    }
                    lr = lr * alpha + psum;
                    for (int d = 0; d < hd; d++) {
                        float a = o[d] * alpha;
                        for (int j = 0; j < 8; j++)
                            if (tt + j < len) a += pv[j] * kv_value(vc[(long)(t0 + tt + j) * kv_stride + kvh * hd + d]);
                        o[d] = a;
                    }
                }
        for (int g = 0; g < G; g++) {
            float mr = wm[g], lr = wl[g];
            float* o = wo.data() + (size_t)g * hd;
            for (int w = 1; w < 4; w++) {
                const float mw = wm[w * G + g];
                if (mw == NEG) continue;
                const float mn = std::max(mr, mw), a = std::exp2(mr - mn), aw = std::exp2(mw - mn);
                lr = lr * a + wl[w * G + g] * aw;
                const float* ow = wo.data() + ((size_t)w * G + g) * hd;
                for (int d = 0; d < hd; d++) o[d] = o[d] * a + ow[d] * aw;
                mr = mn;
            }
            const int h = kvh * G + g;
            if (nsplit == 1) {
                const float f = (1.f / BIAS) / lr;
                for (int d = 0; d < hd; d++) out[(long)b * out_stride + (long)h * hd + d] = o[d] * f;
            } else {
                float* p = P(g);
                for (int d = 0; d < hd; d++) p[d] = o[d] * (1.f / BIAS);
                p[hd] = mr * LN2;
                p[hd + 1] = lr;
            }
        }
    };
    parallel_for((long)n_kv * m * nsplit, threads, block);
    if (nsplit > 1) combine(part.data(), out, out_stride, pos0, m, n_heads, hd, nsplit, want, cap);
}

// ---------------------------------------------------------------- attn_prefill_tc<128> (src/cuda.rs:2408-2617)
// Per query row: Q rounded to f16 after scaling by scale*log2(e); per 32-key tile S = f16 Q . f16 K in f32;
// mask keys past the row's position; running max in base 2; P = f16(exp2(s - m)); l = alpha*l + sum(P);
// O = alpha*O + P V; out = O / l.
// KV_T = int8_t: the KV8 build (src/cuda.rs:2466-2498, 2548-2605): keys staged as exact integers, the score
// times the key's scale; P V takes f16(p * vscale * 2^10) and the row sum the f16-rounded p; out = O / 2^10 / l.
// hd: 128, or 256 (attention_prefill_tc256 = attn_prefill_tc<256, 2>, src/cuda.rs:2623: the same roundings; its
// two blocks per head split the output dims only).
template <typename KV_T>
void prefill_tc(const float* q, long q_stride, const KV_T* kc, const KV_T* vc, const float* ks, const float* vs,
                long kv_stride, float* out, long out_stride, int pos0, int n, int n_heads, int n_kv, float scale,
                int threads, int hd = 128) {
    const int BK = 32, G = n_heads / n_kv;
    const float* W = widen().v;
    const float vbias = ks ? 1024.f : 1.f;
    const float qs = scale * 1.4426950408889634f;
    const int kv_len = pos0 + n;
    auto row_task = [&](long idx) {
        int r = (int)(idx / n_heads), h = (int)(idx % n_heads);
        int kvh = h / G;
        float qh[256], o[256] = {0};
        for (int d = 0; d < hd; d++) qh[d] = W[f32_to_f16(q[(long)r * q_stride + (long)h * hd + d] * qs)];
        int p_row = pos0 + r;
        float m = -std::numeric_limits<float>::infinity(), l = 0.f;
        // the block's key range: its 64-query tile ends at pos0 + q0 + 64 (tiles are still masked per row)
        int kmax = std::min(kv_len, pos0 + (r / 64) * 64 + 64);
        for (int t0 = 0; t0 < kmax; t0 += BK) {
            if (t0 > p_row) break; // every key of the tile is masked for this row: p stays 0, alpha 1
            float s[32], mx = -std::numeric_limits<float>::infinity();
            for (int j = 0; j < BK; j++) {
                int kp = t0 + j;
                if (kp > p_row || kp >= kv_len) { s[j] = -std::numeric_limits<float>::infinity(); continue; }
                const KV_T* kt = kc + (long)kp * kv_stride + kvh * hd;
                float a = 0.f;
                for (int d = 0; d < hd; d++) a += qh[d] * kv_value(kt[d]);
                s[j] = ks ? a * ks[(long)kp * n_kv + kvh] : a;
                mx = std::max(mx, s[j]);
            }
            float mn = std::max(m, mx);
            float alpha = std::exp2(m - mn);
            m = mn;
            float p[32], pv[32], psum = 0.f;
            for (int j = 0; j < BK; j++) {
                const float e = std::exp2(s[j] - mn);
                p[j] = W[f32_to_f16(e)];
                pv[j] = vs && t0 + j < kv_len ? W[f32_to_f16(e * (vs[(long)(t0 + j) * n_kv + kvh] * vbias))] : p[j];
                psum += p[j];
            }
            l = l * alpha + psum;
            for (int d = 0; d < hd; d++) o[d] *= alpha;
            for (int j = 0; j < BK; j++) {
                int kp = t0 + j;
                if (pv[j] == 0.f || kp >= kv_len) continue;
                const KV_T* vt = vc + (long)kp * kv_stride + kvh * hd;
                for (int d = 0; d < hd; d++) o[d] += pv[j] * kv_value(vt[d]);
            }
        }
        float inv = (1.f / vbias) / l;
        for (int d = 0; d < hd; d++) out[(long)r * out_stride + (long)h * hd + d] = o[d] * inv;
    };
    parallel_for((long)n * n_heads, threads, row_task);
}

// kv_store's int8 branch (src/cuda.rs:333-339) for one row.
void kv_quant_i8(const float* src, int hd, int8_t* dst, float* scale) {
    float amax = 0.f;
    for (int d = 0; d < hd; d++) amax = std::max(amax, std::fabs(src[d]));
    const float dd = amax / 127.f, inv = dd != 0.f ? 1.f / dd : 0.f;
    for (int d = 0; d < hd; d++) dst[d] = (int8_t)std::nearbyint(src[d] * inv);
    *scale = dd;
}

// ---------------------------------------------------------------- the 4-bit cache (KV4, src/cuda.rs:226-256)
// kv4_fwht (src/cuda.rs:242-256): the normalized 256-point Walsh-Hadamard transform in Sylvester order, in place.
// Butterfly stages h = 1, 2, ..., 128; within a stage element j (bit h of j clear) and j + h become a + c and
// a - c; then every element times 1/16. Each stage's sums are single f32 additions, so any implementation with
// the same stage order and pairing gives the same bits. hadamard_rows (src/cuda.rs:4675-4693), which rotates
// the attention output back, is the same transform (block 256, no signs; its rsqrtf(256) taken as 1/16).
void kv4_fwht(float* b) {
    for (int h = 1; h < 256; h <<= 1)
        for (int i = 0; i < 128; i++) {
            const int j = (i / h) * 2 * h + (i % h);
            const float a = b[j], c = b[j + h];
            b[j] = a + c;
            b[j + h] = a - c;
        }
    for (int i = 0; i < 256; i++) b[i] *= 0.0625f;
}

// kv_store's KV4 branch (src/cuda.rs:340-357) for one rotated row of 256 values: per group of 32 values
// dh = f16(max|v| / 7) (IEEE division, then round to nearest even), dd = dh as f32, inv = 1/dd (0 when dd is 0),
// q = clamp(rint(v * inv), -7, 7) stored as q + 8; byte i holds values 2i (low nibble) and 2i + 1 (high).
void kv4_quant(const float* v, uint8_t* dst, uint16_t* sc) {
    for (int g = 0; g < 8; g++) {
        float amax = 0.f;
        for (int d = 0; d < 32; d++) amax = std::max(amax, std::fabs(v[32 * g + d]));
        const uint16_t dh = f32_to_f16(amax / 7.f);
        const float dd = f16_to_f32(dh), inv = dd != 0.f ? 1.f / dd : 0.f;
        for (int d = 0; d < 32; d += 2) {
            auto q = [&](float x) { return (unsigned)(std::min(std::max(std::nearbyint(x * inv), -7.f), 7.f) + 8.f); };
            dst[(32 * g + d) / 2] = (uint8_t)(q(v[32 * g + d]) | (q(v[32 * g + d + 1]) << 4));
        }
        sc[g] = dh;
    }
}

// kv4_pair (src/cuda.rs:238-240): the stored nibble n of a group with scale bits s as the f16 f16((n - 8) * s).
uint16_t kv4_value(unsigned n, uint16_t s) { return f32_to_f16((float)((int)n - 8) * f16_to_f32(s)); }

// A 4-bit cache ([rows][n_kv][128] bytes, scales [rows][n_kv][8] f16) as the f16 rows [rows][n_kv * 256] the
// tensor-core kernels stage (src/cuda.rs:2495-2514 for the prefill, 2681-2760 for the decode).
std::vector<uint16_t> kv4_dequant(const uint8_t* c, const uint16_t* sc, long rows, int n_kv) {
    std::vector<uint16_t> out((size_t)rows * n_kv * 256);
    for (long r = 0; r < rows; r++)
        for (int h = 0; h < n_kv; h++) {
            const uint8_t* row = c + ((size_t)r * n_kv + h) * 128;
            const uint16_t* s = sc + ((size_t)r * n_kv + h) * 8;
            uint16_t* o = out.data() + ((size_t)r * n_kv + h) * 256;
            for (int i = 0; i < 128; i++) {
                o[2 * i] = kv4_value(row[i] & 15, s[i / 16]);
                o[2 * i + 1] = kv4_value(row[i] >> 4, s[i / 16]);
            }
        }
    return out;
}

// qk_norm_rope's arithmetic (src/cuda.rs:437-486); store(is_k, pos, kv_head, row) writes a k or v row
// into the cache in its format.
// rotate (the KV4 build, src/cuda.rs:472-479): q and k heads are rotated by kv4_fwht after RoPE (written back
// rotated); the store rotates v rows itself.
template <typename Store>
void qk_norm_rope(float* qkv, const float* qn, const float* kn, int pos0, int n, int n_heads, int n_kv, int hd,
                  int rope_dim, float base, const float* ff, int neox, float eps, Store store, bool rotate = false) {
    const long q_dim = (long)n_heads * hd, kv_dim = (long)n_kv * hd, row_len = q_dim + 2 * kv_dim;
    for (int b = 0; b < n; b++) {
        const int pos = pos0 + b;
        float* row = qkv + b * row_len;
        for (int h = 0; h < n_heads + 2 * n_kv; h++) {
            if (h >= n_heads + n_kv) {
                const int vh = h - n_heads - n_kv;
                store(0, pos, vh, row + q_dim + kv_dim + (long)vh * hd);
                continue;
            }
            float* vec = row + (long)h * hd;
            if (qn) {
                const float* w = h < n_heads ? qn : kn;
                float ss = 0.f;
                for (int d = 0; d < hd; d++) ss += vec[d] * vec[d];
                const float scale = 1.0f / std::sqrt(ss / (float)hd + eps);
                for (int d = 0; d < hd; d++) vec[d] = vec[d] * scale * w[d];
            }
            const int half = rope_dim / 2;
            for (int i = 0; i < half; i++) {
                float freq = std::pow(base, -2.0f * (float)i / (float)rope_dim);
                if (ff) freq /= ff[i];
                const float ang = (float)pos * freq;
                const float s = std::sin(ang), c = std::cos(ang);
                const int ia = neox ? i : 2 * i, ib = neox ? i + half : 2 * i + 1;
                const float x = vec[ia], y = vec[ib];
                vec[ia] = x * c - y * s;
                vec[ib] = x * s + y * c;
            }
            if (rotate) kv4_fwht(vec);
            if (h >= n_heads) store(1, pos, h - n_heads, vec);
        }
    }
}


} // namespace

extern "C" {

float gio_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t gio_f32_to_f16(float f) { return f32_to_f16(f); }

void gio_f16_to_f32_array(const uint16_t* src, float* dst, size_t count) {
    const float* w = widen().v;
    for (size_t i = 0; i < count; i++) dst[i] = w[src[i]];
}
void gio_f32_to_f16_array(const float* src, uint16_t* dst, size_t count) {
    for (size_t i = 0; i < count; i++) dst[i] = f32_to_f16(src[i]);
}

float gio_dot_f32(const float* a, const float* b, int n) { return dot_f32(a, b, n); }

// att_want (src/cuda.rs:8426-8428) for the grouped-query kernel: ceil(96 / n_kv)
int gio_att_want(int n_kv) { return (ATT_TARGET_BLOCKS + n_kv - 1) / n_kv; }
int gio_att_chunk(int span, int want, int cap) { return att_chunk(span, want, cap); }
// max_splits (src/cuda.rs:8441-8444): most slices any span 1..=ctx needs
int gio_max_splits(int ctx, int want, int cap) {
    int best = 1;
    for (int span = 1; span <= ctx; span++) best = std::max(best, (span + att_chunk(span, want, cap) - 1) / att_chunk(span, want, cap));
    return best;
}

// Model::attention over an f32 cache. q: [n][q_stride] (the query heads at the start of each row),
// caches [pos][kv_stride] with kv head h at h*hd, out [n][out_stride]. threads = the worker count
// (rayon's current_num_threads), which also fixes the split count.
void gio_attention_f32(const float* q, long q_stride, const float* kc, const float* vc, long kv_stride, float* out,
                       long out_stride, int pos0, int n, int n_heads, int n_kv, int hd, float scale, int threads) {
    Cache k, v;
    k.f32 = kc; v.f32 = vc; k.stride = v.stride = kv_stride;
    model_attention(q, q_stride, k, v, out, out_stride, pos0, n, n_heads, n_kv, hd, scale, threads);
}

// The same over an f16 cache, each row widened exactly to f32 as it is read (the reference caches f32 on
// the CPU; the widening is exact, so this equals gio_attention_f32 on the widened cache).
void gio_attention_f16kv(const float* q, long q_stride, const uint16_t* kc, const uint16_t* vc, long kv_stride,
                         float* out, long out_stride, int pos0, int n, int n_heads, int n_kv, int hd, float scale,
                         int threads) {
    Cache k, v;
    k.f16 = kc; v.f16 = vc; k.stride = v.stride = kv_stride;
    model_attention(q, q_stride, k, v, out, out_stride, pos0, n, n_heads, n_kv, hd, scale, threads);
}

// attention_partial_gqa + attention_combine semantics for m tokens (head size 128, f16 cache). nsplit,
// want and cap as the reference's host computes them (gio_att_want, gio_max_splits, cap 128).
void gio_decode_gpu(const float* qkv, long q_stride, const uint16_t* kc, const uint16_t* vc, long kv_stride, float* out,
                    long out_stride, int pos0, int m, int n_heads, int n_kv, float scale, int nsplit, int want, int cap,
                    int threads) {
    decode_gpu<uint16_t>(qkv, q_stride, kc, vc, nullptr, nullptr, kv_stride, out, out_stride, pos0, m, n_heads, n_kv,
                         scale, nsplit, want, cap, threads);
}

// The same with the int8 cache (KV8): kc / vc int8 rows, ks / vs f32 scales [pos][n_kv].
void gio_decode_gpu_i8(const float* qkv, long q_stride, const int8_t* kc, const int8_t* vc, const float* ks,
                       const float* vs, long kv_stride, float* out, long out_stride, int pos0, int m, int n_heads,
                       int n_kv, float scale, int nsplit, int want, int cap, int threads) {
    decode_gpu<int8_t>(qkv, q_stride, kc, vc, ks, vs, kv_stride, out, out_stride, pos0, m, n_heads, n_kv, scale, nsplit,
                       want, cap, threads);
}

// kv_store with KV8 (src/cuda.rs:333-339) over `rows` rows of hd values: dd = max|x| / 127, each value
// rint(x * (1/dd)) as int8 (0 when dd is 0), dd to the row's scale. Division correctly rounded, rint to
// nearest even (the reference's IEEE `/` and __float2int_rn).
void gio_decode_tc256_i8(const float* qkv, long q_stride, const int8_t* kc, const int8_t* vc, const float* ks,
                         const float* vs, long kv_stride, float* out, long out_stride, int pos0, int m, int n_heads,
                         int n_kv, float scale, int nsplit, int want, int cap, int threads) {
    decode_tc256<int8_t>(qkv, q_stride, kc, vc, ks, vs, kv_stride, out, out_stride, pos0, m, n_heads, n_kv, scale,
                         nsplit, want, cap, threads);
}

void gio_kv_quant_i8(const float* src, long rows, int hd, int8_t* dst, float* scales) {
    for (long r = 0; r < rows; r++) kv_quant_i8(src + r * hd, hd, dst + r * hd, scales + r);
}

// attn_prefill_tc<128> semantics (f16 rounding of the scaled Q and of P).
void gio_prefill_tc(const float* q, long q_stride, const uint16_t* kc, const uint16_t* vc, long kv_stride, float* out,
                    long out_stride, int pos0, int n, int n_heads, int n_kv, float scale, int threads) {
    prefill_tc<uint16_t>(q, q_stride, kc, vc, nullptr, nullptr, kv_stride, out, out_stride, pos0, n, n_heads, n_kv, scale,
                         threads);
}

// attn_prefill_tc<256, 2> (f16 cache, head size 256): kv_stride in elements, rows of hd = 256.
void gio_prefill_tc256(const float* q, long q_stride, const uint16_t* kc, const uint16_t* vc, long kv_stride, float* out,
                       long out_stride, int pos0, int n, int n_heads, int n_kv, float scale, int threads) {
    prefill_tc<uint16_t>(q, q_stride, kc, vc, nullptr, nullptr, kv_stride, out, out_stride, pos0, n, n_heads, n_kv, scale,
                         threads, 256);
}

// attn_prefill_tc<128> with the KV8 cache: kc / vc int8 rows, ks / vs f32 scales [pos][n_kv].
void gio_prefill_tc_i8(const float* q, long q_stride, const int8_t* kc, const int8_t* vc, const float* ks,
                       const float* vs, long kv_stride, float* out, long out_stride, int pos0, int n, int n_heads,
                       int n_kv, float scale, int threads) {
    prefill_tc<int8_t>(q, q_stride, kc, vc, ks, vs, kv_stride, out, out_stride, pos0, n, n_heads, n_kv, scale, threads);
}

// attn_prefill_tc<64> (attention_prefill_tc64, src/cuda.rs:2620): gio_prefill_tc's arithmetic at head size 64, over
// the f16 and the KV8 cache.
void gio_prefill_tc64(const float* q, long q_stride, const uint16_t* kc, const uint16_t* vc, long kv_stride, float* out,
                      long out_stride, int pos0, int n, int n_heads, int n_kv, float scale, int threads) {
    prefill_tc<uint16_t>(q, q_stride, kc, vc, nullptr, nullptr, kv_stride, out, out_stride, pos0, n, n_heads, n_kv, scale,
                         threads, 64);
}
void gio_prefill_tc64_i8(const float* q, long q_stride, const int8_t* kc, const int8_t* vc, const float* ks,
                         const float* vs, long kv_stride, float* out, long out_stride, int pos0, int n, int n_heads,
                         int n_kv, float scale, int threads) {
    prefill_tc<int8_t>(q, q_stride, kc, vc, ks, vs, kv_stride, out, out_stride, pos0, n, n_heads, n_kv, scale, threads,
                       64);
}

// attention_prefill_tc256 with KV8 (attn_prefill_tc<256, 2>, src/cuda.rs:2623): gio_prefill_tc_i8's arithmetic at
// head size 256.
void gio_prefill_tc256_i8(const float* q, long q_stride, const int8_t* kc, const int8_t* vc, const float* ks,
                          const float* vs, long kv_stride, float* out, long out_stride, int pos0, int n, int n_heads,
                          int n_kv, float scale, int threads) {
    prefill_tc<int8_t>(q, q_stride, kc, vc, ks, vs, kv_stride, out, out_stride, pos0, n, n_heads, n_kv, scale, threads,
                       256);
}

// qk_norm_rope storing into an int8 cache (kv_store with KV8, src/cuda.rs:333-339): kc / vc int8 rows in the
// element layout of gio_qk_norm_rope, scales at ks / vs [pos*sc_stride + h*sc_head_stride].
void gio_qk_norm_rope_i8(float* qkv, const float* qn, const float* kn, int8_t* kc, int8_t* vc, float* ks, float* vs,
                         long kv_stride, long kv_head_stride, long sc_stride, long sc_head_stride, int pos0, int n,
                         int n_heads, int n_kv, int hd, int rope_dim, float base, const float* ff, int neox, float eps) {
    qk_norm_rope(qkv, qn, kn, pos0, n, n_heads, n_kv, hd, rope_dim, base, ff, neox, eps,
                 [&](int is_k, int pos, int h, const float* src) {
                     const long off = (long)pos * kv_stride + (long)h * kv_head_stride;
                     float* sc = (is_k ? ks : vs) + (long)pos * sc_stride + (long)h * sc_head_stride;
                     kv_quant_i8(src, hd, (is_k ? kc : vc) + off, sc);
                 });
}

// Reference: qk_norm_rope (src/cuda.rs:437-486), f16 cache. qkv rows [q | k | v] f32 are updated in place
// (q and k heads normalised and rotated); k and v heads are stored into kc / vc (f16 bits, RNE). Sums in
// index order; 1/sqrt correctly rounded (the reference's rsqrtf is an approximation of it).
void gio_qk_norm_rope(float* qkv, const float* qn, const float* kn, uint16_t* kc, uint16_t* vc, long kv_stride,
                      long kv_head_stride, int pos0, int n, int n_heads, int n_kv, int hd, int rope_dim, float base,
                      const float* ff, int neox, float eps) {
    qk_norm_rope(qkv, qn, kn, pos0, n, n_heads, n_kv, hd, rope_dim, base, ff, neox, eps,
                 [&](int is_k, int pos, int h, const float* src) {
                     uint16_t* dst = (is_k ? kc : vc) + (long)pos * kv_stride + (long)h * kv_head_stride;
                     for (int d = 0; d < hd; d++) dst[d] = f32_to_f16(src[d]);
                 });
}

// kv4_fwht over `rows` rows of 256 values, in place (also hadamard_rows with block 256).
void gio_kv4_fwht(float* x, long rows) {
    for (long r = 0; r < rows; r++) kv4_fwht(x + r * 256);
}

// kv_store's KV4 branch over `rows` already-rotated rows of 256 values: dst 128 bytes a row, sc 8 f16 a row.
void gio_kv4_quant(const float* src, long rows, uint8_t* dst, uint16_t* sc) {
    for (long r = 0; r < rows; r++) kv4_quant(src + r * 256, dst + r * 128, sc + r * 8);
}

// The f16 values the kernels use for a 4-bit cache of `rows` rows (reference layout, n_kv heads a row).
void gio_kv4_dequant(const uint8_t* c, const uint16_t* sc, long rows, int n_kv, uint16_t* out) {
    std::vector<uint16_t> v = kv4_dequant(c, sc, rows, n_kv);
    std::memcpy(out, v.data(), v.size() * sizeof(uint16_t));
}

// qk_norm_rope with the KV4 build (src/cuda.rs:437-486, 340-357): q and k heads rotated after RoPE, the k row
// quantised as it is, a v row rotated and then quantised. Head size 256; the cache in the reference layout
// (kc / vc [pos][n_kv][128] bytes, ks / vs [pos][n_kv][8] f16).
void gio_qk_norm_rope_q4(float* qkv, const float* qn, const float* kn, uint8_t* kc, uint8_t* vc, uint16_t* ks,
                         uint16_t* vs, int pos0, int n, int n_heads, int n_kv, int rope_dim, float base,
                         const float* ff, int neox, float eps) {
    qk_norm_rope(qkv, qn, kn, pos0, n, n_heads, n_kv, 256, rope_dim, base, ff, neox, eps,
                 [&](int is_k, int pos, int h, const float* src) {
                     float row[256];
                     std::memcpy(row, src, sizeof row);
                     if (!is_k) kv4_fwht(row);
                     const long r = (long)pos * n_kv + h;
                     kv4_quant(row, (is_k ? kc : vc) + r * 128, (is_k ? ks : vs) + r * 8);
                 },
                 true);
}

// attention_decode_tc256 with the KV4 build + attention_combine: the 4-bit cache dequantised to the f16
// fragments, unit scales, P = f16(p * 2^10). q rows are the rotated queries; out is rotated (hadamard_rows
// turns it back). rows: positions the cache holds (at least pos0 + m).
void gio_decode_tc256_q4(const float* qkv, long q_stride, const uint8_t* kc, const uint8_t* vc, const uint16_t* ks,
                         const uint16_t* vs, long rows, float* out, long out_stride, int pos0, int m, int n_heads,
                         int n_kv, float scale, int nsplit, int want, int cap, int threads) {
    std::vector<uint16_t> kh = kv4_dequant(kc, ks, rows, n_kv), vh = kv4_dequant(vc, vs, rows, n_kv);
    decode_tc256<uint16_t>(qkv, q_stride, kh.data(), vh.data(), nullptr, nullptr, (long)n_kv * 256, out, out_stride,
                           pos0, m, n_heads, n_kv, scale, nsplit, want, cap, threads);
}

// attention_prefill_tc256 with the KV4 build (src/cuda.rs:2495-2514): the tiles staged as the f16 values of the
// 4-bit cache, then the f16 cache's arithmetic (P = f16(p), out = O / l).
void gio_prefill_tc256_q4(const float* q, long q_stride, const uint8_t* kc, const uint8_t* vc, const uint16_t* ks,
                          const uint16_t* vs, long rows, float* out, long out_stride, int pos0, int n, int n_heads,
                          int n_kv, float scale, int threads) {
    std::vector<uint16_t> kh = kv4_dequant(kc, ks, rows, n_kv), vh = kv4_dequant(vc, vs, rows, n_kv);
    prefill_tc<uint16_t>(q, q_stride, kh.data(), vh.data(), nullptr, nullptr, (long)n_kv * 256, out, out_stride, pos0,
                         n, n_heads, n_kv, scale, threads, 256);
}

} // extern "C"
