// Attention kernels for CDNA4 (gfx950): split-K flash decoding and causal flash prefill over a
// grouped-query f16 KV cache. Built offline into a code object (gi_attn_gfx950.hsaco) that the C-ABI
// library (gi_attn_host.cpp) loads with hipModuleLoad and launches by name.
//
// Cache layout: K and V are separate f16 buffers; key/value t of kv head h starts at element
// t*kv_stride + h*kv_head_stride. The reference's layout (src/cuda.rs:365-369, src/cuda.rs:10229-10242) is
// [position][kv head][128] (kv_stride = n_kv*128, kv_head_stride = 128); the head-major layout
// [kv head][position][128] (kv_stride = 128, kv_head_stride = capacity*128) keeps each head contiguous,
// which streams evenly over the HBM channels.
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
// Prefill (reference semantics: attn_prefill_tc<128>, src/cuda.rs:2408-2617: Q*scale*log2(e) rounded to
// f16, base-2 online softmax, P rounded to f16, the row sum taken over the rounded P). Defined further
// below.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef _Float16 h4x __attribute__((ext_vector_type(4)));

#define GI_NEG_INF (-__builtin_inff())
#define GI_LOG2E 1.4426950408889634f

// ------------------------------------------------------------------------------------------------ decode

// Arguments of the decode kernels (one struct so the host and the device agree on one definition).
struct GiDecodeArgs {
    const float* q;        // query rows: token b's head h at q + b*q_stride + h*128 (f32)
    const uint16_t* kc;    // K cache [pos][n_kv][128] f16, kv_stride elements per position
    const uint16_t* vc;    // V cache, same layout
    float* part;           // slice partials [token][head][nsplit][hd + 4]: O (hd), max (base 2), sum, 2 pad
    float* out;            // output rows: token b's head h at out + b*out_stride + h*128 (f32)
    const int* posp;       // device position (overrides pos0 when non-null)
    long long q_stride;
    long long kv_stride;
    long long out_stride;
    long long kv_head_stride;
    int pos0;              // position of token 0: token b attends to keys 0..pos0+b
    int n_tok;
    int n_heads;
    int n_kv;
    int chunk;             // keys per slice: whole wave tiles, at least one per wave
    int nsplit;            // slices per token (the grid's x)
    float qscale;          // scale * log2(e)
    int hd;                // head size: 128 or 256 (f16 cache); partial rows are hd + 4 floats
    // int8 cache only (the kernels named *_i8): kc / vc hold int8 rows in the same element layout, and the
    // f32 scale of position t, kv head h is at ks / vs [t*sc_stride + h*sc_head_stride]. The 4-bit cache (*_q4):
    // kc / vc rows of 128 bytes with kv_stride / kv_head_stride in bytes, ks / vs the rows' 8 f16 scales with
    // sc_stride / sc_head_stride in f16 elements
    const float* ks;
    const float* vs;
    long long sc_stride;
    long long sc_head_stride;
    int kv_cap;            // with posp: keys the cache holds; *posp is clamped to [0, kv_cap - n_tok]
    int pad_;
};

// Slice partials of gi_attn_decode_noalloc: a module-global array (one per device, since every device loads
// the code object itself), for callers that cannot allocate a workspace. Calls on one device share it.
#define GI_SCRATCH_BYTES (16u << 20)
__device__ __attribute__((used, aligned(256))) unsigned char gi_scratch[GI_SCRATCH_BYTES];

#define DEC_WAVES 4
#ifndef DEC_NB
#define DEC_NB 2 // register buffers of K/V tiles per wave (tiles in flight)
#endif
#ifndef DEC_XCD_GROUPS // pair groups of one slice on one XCD
#define DEC_XCD_GROUPS 1
#endif
#ifndef DEC_MINWG
#define DEC_MINWG 1 // workgroups per CU the register budget is sized for
#endif
#define DEC_TILE 32
// An empty volatile asm: a block holding it cannot be executed speculatively, so the compiler keeps the
// (wave-uniform) branch around it instead of turning the block into selects that run every time.
#define GI_KEEP_BRANCH() asm volatile("")
#ifndef DEC_PIPE // software-pipelined tiles in the one-pair-per-column f16 kernels
#define DEC_PIPE 1
#endif
#ifndef DEC_CPOL // cache policy of the K/V loads of decode variants whose waves stream tiles of their own (2: nt)
#define DEC_CPOL 2
#endif
#define DEC_PAIRS 8 // (token, head) pairs per column block of 16 columns
#ifndef DEC_V256_DENSE // f16 cache, head size 256: each V load instruction reads whole 256-byte runs of a row
#define DEC_V256_DENSE 1
#endif
#ifndef DEC_I8_MFMA // int8 cache, up to 8 pairs (hi/lo columns): QK on int8 MFMA against the query's int8 limbs
#define DEC_I8_MFMA 1
#endif
typedef int i4v __attribute__((ext_vector_type(4)));
#define DEC_RESCALE_LOG2 8.0f
// int8 cache: the probability's f16 remainder column is scaled by 2^12 (undone when the columns merge).
// Times a value scale of ~0.03 the remainder would otherwise fall into f16's subnormal range.
#define DEC_I8_LO 4096.f
// (with one pair per column the high and remainder parts share an accumulator, so P times the value scale is
// biased as a whole instead; the merge divides it out)
#define DEC_I8_VB 64.f
// Head size 256 over the int8 and 4-bit caches (the reference's attention_decode_tc256, src/cuda.rs:2625-2802):
// one f16 Q (Q*scale*log2e rounded once) and one f16 P (p times the value scale and a bias, rounded once), the
// reference's own roundings, with the exp-sum of the unrounded p. The reference biases by 2^10 with p <= 1; here p
// <= 2^8 (the lazy rescale), so the bias is 4: the same largest P for a given value scale.
#define DEC_REF_VB 4.f
#define GI_RSRC_FLAGS 0x00020000

__device__ __forceinline__ float wave_xor(float v, int m) { return __shfl_xor(v, m, 64); }
// Scales an MFMA accumulator (held in AGPRs) by alpha in the rare rescale branch of an online softmax. The empty
// asm statements pin the accumulator to AGPRs on both sides of the multiply, so the AGPR -> VGPR copies it needs are
// made inside the branch; without them the compiler hoists those copies into every tile iteration (up to 135
// accvgpr reads per tile in the head-256 4-bit verify, all dead unless the branch is taken).
// PIN = false: kernels whose accumulators the compiler keeps in VGPRs (the prefill's two waves per SIMD and the
// short-span decode), where the pin would move them into AGPRs and spill.
template <bool PIN, typename T> __device__ __forceinline__ void gi_acc_scale(T& acc, float alpha) {
    if constexpr (PIN) asm volatile("" : "+a"(acc));
    acc *= alpha;
    if constexpr (PIN) asm volatile("" : "+a"(acc));
}
// v of lane l ^ 1 (DPP quad permutation, no LDS round trip)
__device__ __forceinline__ float lane_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
}
// max / sum of v over lanes l, l^16, l^32, l^48 (the four 16-lane rows), left in every lane: the
// permlane swaps pair row r of one copy with row r^2 (32-swap) or r^1 (16-swap) of the other
__device__ __forceinline__ float rows_max(float v) {
    auto p = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    v = fmaxf(__int_as_float(p[0]), __int_as_float(p[1]));
    auto q = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
    return fmaxf(__int_as_float(q[0]), __int_as_float(q[1]));
}
__device__ __forceinline__ float rows_sum(float v) {
    auto p = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    v = __int_as_float(p[0]) + __int_as_float(p[1]);
    auto q = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
    return __int_as_float(q[0]) + __int_as_float(q[1]);
}

// Buffer resource over `bytes` bytes from p: loads at offsets >= bytes return zeros without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gi_rsrc(const void* p, long long bytes) {
    int n = (int)(bytes < 0 ? 0 : (bytes > 0x7ffffff0ll ? 0x7ffffff0ll : bytes));
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, n, GI_RSRC_FLAGS);
}
__device__ __forceinline__ u4 gi_load16(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u2 gi_load8(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
// Loads with an explicit cache policy: 2 is `nt` on gfx950 (streaming: the line leaves the caches first),
// for data no other wave reads again.
template <int CPOL> __device__ __forceinline__ u4 gi_load16p(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CPOL);
}
template <int CPOL> __device__ __forceinline__ u2 gi_load8p(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CPOL);
}
__device__ __forceinline__ float gi_load4f(__amdgpu_buffer_rsrc_t r, int off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// int8 -> f16, exactly, two bytes of x (bytes 0-1 for GI_I8_LO, 2-3 for GI_I8_HI) into one f16 pair. With its
// sign bit flipped a byte is u = v + 128 in 0..255; the f16 with bits 0x6400 | u is 1024 + u, so subtracting
// 1152 leaves v. x holds 4 bytes already flipped (gi_i8_in), and v_perm picks bytes of {0x64646464 : x}
// (selector bytes 0-3 take x, 4-7 the constant): one v_perm and one packed f16 subtract per two values. Every
// instruction is visible to the compiler, which must see the writes that feed an MFMA operand to keep the
// required wait states (a conversion by inline asm right before an MFMA reading its result was measured to
// lose values).
typedef _Float16 h2x __attribute__((ext_vector_type(2)));
#define GI_I8_LO 0x04010400u // bytes 0, 1 of x -> f16 pair
#define GI_I8_HI 0x04030402u // bytes 2, 3
__device__ __forceinline__ uint32_t gi_i8_in(uint32_t x) { return x ^ 0x80808080u; }
__device__ __forceinline__ uint32_t i8_f16x2(uint32_t x, uint32_t sel) {
    const h2x v = __builtin_bit_cast(h2x, __builtin_amdgcn_perm(0x64646464u, x, sel)) -
                  h2x{(_Float16)1152.f, (_Float16)1152.f};
    return __builtin_bit_cast(uint32_t, v);
}
// v of lane 16*(l/16) + m: the lane's 16-lane row broadcasts its m-th lane (DPP row_newbcast)
template <int M>
__device__ __forceinline__ float row_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + M, 0xF, 0xF, false));
}

// Register buffers of one wave's tile. f16: 32 keys; K as the S^T A operand (2 blocks of 16 keys, 4 k-steps
// of 32 dims), V as 8 keys x 8 dims. int8: 64 keys in the same registers; K 4 blocks x 32 bytes, V 16 keys x
// 8 dims, plus the scale of key `lane` of the tile.
template <bool I8, int HD> struct DecBuf { u4 k[2][4]; u4 v[8]; };
template <> struct DecBuf<true, 128> { u4 k[4][2]; u2 v[16]; float ksc, vsc; };
// head size 64: the head-128 tiles with half the K k-steps; V 8 keys x 4 dims (4c..4c+3) as f16, 16 keys x 4 dims
// as int8 (the second word unused)
template <> struct DecBuf<false, 64> { u4 k[2][2]; u2 v[8]; };
template <> struct DecBuf<true, 64> { u4 k[4][1]; u2 v[16]; float ksc, vsc; };
// head size 256 (f16): 16 keys; K row c of the tile, 8 k-steps of 32 dims; V keys 4grp..4grp+3, dims 16c..16c+15
template <> struct DecBuf<false, 256> { u4 k[8]; u4 v[4][2]; };
// head size 256 over the int8 cache: 16 keys; K row c, bytes 64i + 16grp .. +15 (k-steps 2i, 2i + 1); V keys
// 4grp..4grp+3, bytes 16c..16c+15; the scales of tile key 4(lane/16) + lane%4
template <> struct DecBuf<true, 256> { u4 k[4]; u4 v[4]; float ksc, vsc; };
// head size 256 over the 4-bit cache: 16 keys; K row c, bytes 32grp .. 32grp + 31 (values 64grp .. 64grp + 63,
// scale groups 2grp and 2grp + 1, both scales in ksc); V keys 4grp + i, bytes 8c .. 8c + 7 (dims 16c .. 16c + 15,
// scale group c/2, that scale in vsc[i])
struct DecBufQ4 { u4 k[2]; u2 v[4]; uint32_t ksc; uint32_t vsc[4]; };
template <typename T, int N> __device__ __forceinline__ void gi_touch(T (&k)[N]) {
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" ::"v"(k[i]));
}
template <typename T, int N, int M> __device__ __forceinline__ void gi_touch(T (&k)[N][M]) {
#pragma unroll
    for (int i = 0; i < N; i++) gi_touch(k[i]);
}
template <bool C, typename A, typename B> struct gi_pick { typedef A type; };
template <typename A, typename B> struct gi_pick<false, A, B> { typedef B type; };

// 4-bit cache values -> f16 (kv4_pair, src/cuda.rs:238-240: f16((n - 8) * s)). lo and hi hold, in byte j, the
// nibbles that become the low and high f16 of the pair; v_perm puts byte j of each into the low byte of a half,
// the and-or keeps the nibbles under the f16 bits 0x6400 (1024 + n), the packed subtract leaves n - 8 exactly
// and the packed multiply by the scales rounds (n - 8) * s to nearest even once, as the reference's conversion
// of the exact f32 product does.
__device__ __forceinline__ uint32_t q4_f16x2(uint32_t hi, uint32_t lo, int j, h2x sc) {
    const uint32_t sel = (uint32_t)j | 0x0c00u | (uint32_t)(4 + j) << 16 | 0x0c000000u;
    const uint32_t w = (__builtin_amdgcn_perm(hi, lo, sel) & 0x000f000fu) | 0x64006400u;
    const h2x v = (__builtin_bit_cast(h2x, w) - h2x{(_Float16)1032.f, (_Float16)1032.f}) * sc;
    return __builtin_bit_cast(uint32_t, v);
}

// Lane l of a wave: c = l % 16 (MFMA column / A-row), grp = l / 16 (k-group of 8).
// I8 = true: an int8 cache (kv_store's KV8 format, src/cuda.rs:333-339: a row of int8 values and one f32
// scale per (position, kv head)). Scores are attention_partial_gqa's (src/cuda.rs:1750-1760): the dot
// product with the integer key, times the key's scale; the value scale rides on the probability
// (src/cuda.rs:1812-1822) and the exp-sum is of the unscaled probabilities. Value bytes are widened to exact f16
// in registers for the f16 P V MFMA; key bytes too where the query takes two f16 columns a pair (one pair per
// column), and otherwise QK runs on int8 MFMA against the query's integer limbs (I8M below). Tiles are 64 keys (the same register bytes as 32
// f16 keys); lane (c, grp) holds the S^T rows of keys 16grp + 4b + j (block b, row 4grp + j, so A-row c of
// block b loads key 16(c/4) + c%4 + 4b) and feeds PV with V rows 16grp..16grp+15 (k-step ks: 8ks..8ks+7),
// dims 8c..8c+7. Each key's scale is loaded by lane key%64 and broadcast across its 16-lane row.
// HD = 256 (f16 cache): tiles of 16 keys (16 KB of K and V, as before). S^T comes from 8 k-steps of
// v_mfma_f32_16x16x32_f16 with A-row c = tile key c; lane (c, grp) then holds the scores of keys 4grp..4grp+3,
// exactly the B operand of v_mfma_f32_16x16x16_f16 for O^T += V^T P^T over the tile, so no key permutation
// is needed. V^T block dd has A-row c = dim 16c + dd (the lane loads dims 16c..16c+15 of its 4 keys), so a
// lane ends with dims 64grp..64grp+63 of its column.
// PM = true (head size 128, blocks of more than 8 pairs): one (token, head) pair per column, 16 per column
// block; the f16 high part and remainder of Q and of P are separate MFMAs into the same accumulator instead
// of neighbouring columns, so a lane's softmax serves one pair and no lane repeats its neighbour's (half the
// VALU per pair; twice the MFMAs per column, so blocks of at most 8 pairs keep PM = false).
// WS (waves per pair set) = 4: the 4 waves split the slice's tiles and serve the same DEC_PAIRS*NCB (token, head)
// pairs, merging through LDS at the end. WS = 2 (many pairs per kv head, as in a verify block): waves 2p and
// 2p + 1 split the tiles for pair set p, so one workgroup serves two sets and each tile's second read comes
// from the caches of the same CU.
// Q4 = true (head size 256, the 4-bit cache, kv_store's KV4 format, src/cuda.rs:340-357): K and V values are
// widened to the f16 values f16((n - 8) * scale) that attention_decode_tc256 (src/cuda.rs:2681-2760) feeds its
// tensor cores, and the rest is the f16 cache's path (unit key and value scales). Lane (c, grp) takes values
// 64grp .. 64grp + 63 of key row c (k-step kk: 64grp + 8kk .. + 7, the query loaded to match), so each lane's two
// 16-byte loads are whole scale groups.
// F32 = true (head size 256 over the int8 cache): f32 precision through the f16 high/remainder split, as at the
// other head sizes, instead of the tc256 roundings: the reference's attention_partial_gqa hd-256 branch
// (src/cuda.rs:1762-1781), which serves this cache when its tensor-core decode is off (GHOST_INFER_NO_TC_ATT or
// GHOST_INFER_NO_TC_DECODE, src/cuda.rs:5655).
// NBO: tiles in flight per wave when nonzero (the short-span kernel: one, since each wave then has a tile or two)
template <int NCB, int WS, bool I8, int HD = 128, bool PM = false, bool Q4 = false, bool F32 = false, int NBO = 0>
__device__ __forceinline__ void gi_decode_partial_t(GiDecodeArgs a) {
    static_assert(HD == 64 || HD == 128 || HD == 256, "head sizes: 64, 128, 256");
    static_assert(!Q4 || (HD == 256 && !I8), "the 4-bit cache: head size 256");
    static_assert(!F32 || (I8 && HD == 256), "the f32-precise form: head size 256 over the int8 cache");
    // the reference's tc256 arithmetic (one f16 Q, one f16 P; see DEC_REF_VB): head size 256 over the int8 and
    // 4-bit caches, which these kernels serve with one pair per column
    constexpr bool REF = (I8 || Q4) && HD == 256 && !F32;
    static_assert(!REF || PM, "head size 256 over the int8 and 4-bit caches: one pair per column");
    // the bias on P that the merge divides out
    constexpr float PBIAS = REF && I8 ? DEC_REF_VB : I8 && PM ? DEC_I8_VB : 1.f;
    // tiles in flight per wave: an int8 tile at head size 256 holds half the bytes of the others (4-bit: a quarter)
    constexpr int NB = NBO ? NBO : (I8 || Q4) && HD == 256 ? 2 * DEC_NB : DEC_NB;
    constexpr int CPAIRS = PM ? 2 * DEC_PAIRS : DEC_PAIRS; // pairs per column block
    constexpr int TILE = HD == 256 ? DEC_TILE / 2 : I8 ? 2 * DEC_TILE : DEC_TILE; // keys per wave tile
    constexpr int KK = HD / 32;                 // QK k-steps
    constexpr int ND = HD / 16;                 // O^T MFMA blocks
    constexpr int PART = HD + 4;                // floats per slice partial
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, grp = lane >> 4;
    // workgroup -> (slice s, kv head, pair group gz). With several pair groups, the groups of one (slice, kv head)
    // take linear ids 8 apart: workgroups go to the 8 XCDs round-robin, so they run on one XCD at about the same
    // time and the later ones find the slice's K/V in that XCD's L2. The (slice, kv head) items past the last
    // whole 8 take the ids left at the end, in plain order.
    int s = blockIdx.x, kvh = blockIdx.y, gz = blockIdx.z;
    if (DEC_XCD_GROUPS && gridDim.z > 1) {
        const int lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
        const int items = gridDim.x * gridDim.y, full = items & ~7;
        int sk; // (slice, kv head) index
        if (lin < full * (int)gridDim.z) {
            gz = (lin >> 3) % gridDim.z;
            sk = (lin / (8 * gridDim.z)) * 8 + (lin & 7);
        } else {
            const int r = lin - full * gridDim.z, tail = items - full;
            gz = r / tail;
            sk = full + r % tail;
        }
        s = sk % gridDim.x;
        kvh = sk / gridDim.x;
    }
    // a device position is clamped so that no key past the cache's capacity is read
    const int pos0 = a.posp ? min(max(*a.posp, 0), a.kv_cap - a.n_tok) : a.pos0;
    const int G = a.n_heads / a.n_kv;
    const int npairs = a.n_tok * G;
    static_assert(WS == 2 || WS == DEC_WAVES, "waves per pair set: 2 or all");
    constexpr int WG_PAIRS = (DEC_WAVES / WS) * CPAIRS * NCB; // pairs per workgroup
    const int pair0 = gz * WG_PAIRS + (wave / WS) * CPAIRS * NCB; // this wave's first pair
    const int kv_len = pos0 + a.n_tok; // keys any token of the launch may see
    const int k_begin = s * a.chunk;
    const int nkeys = min(a.chunk, kv_len - k_begin); // keys of this slice (<= 0: an empty slice)

    // this lane's column(s): pair and hi/lo half; span of the pair's token, relative to the slice
    int span[NCB], qoff[NCB];
    bool valid[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
        int pi = pair0 + cb * CPAIRS + (PM ? c : c >> 1);
        valid[cb] = pi < npairs;
        int t = valid[cb] ? pi / G : 0, g = valid[cb] ? pi % G : 0;
        span[cb] = valid[cb] ? min(pos0 + t + 1 - k_begin, nkeys) : 0; // keys of the slice this column sees
        qoff[cb] = ((int)(t * a.q_stride) + (kvh * G + g) * HD + (Q4 ? 64 : I8 ? 16 : 8) * grp) * 4;
    }
    // smallest span among the wave's valid columns (the lowest token's: column 0 of block 0 is always valid):
    // tiles below it need no masking
    // (the pipelined kernels hold it in an SGPR, which keeps their loop uniform; the others measured 1% faster
    // at config 2 when the compiler places it)
    const int span_lo0 = min(pos0 + pair0 / G + 1 - k_begin, nkeys);
    const int span_lo = PM ? __builtin_amdgcn_readfirstlane(span_lo0) : span_lo0;
    // Q rows (f32, 8 dims per lane per k-step), issued before the first K/V tiles so that waiting for them
    // leaves the K/V loads in flight
    u4 qraw[NCB][KK][2];
    // B operand of S^T = K Qc^T. f16: k-step kk covers dims 32kk..32kk+31, this lane dims 32kk+8grp..+7.
    // int8: this lane dims 16grp + 8(kk%2) + 64(kk/2) .. +7 (the bytes its two 16-byte key loads bring)
    h8 qf[NCB][KK];
    h8 qfl[NCB][REF ? 1 : KK]; // PM: the remainders (REF: none; else unused)
    // I8M: the int8 cache with up to 8 pairs at head sizes 64 and 128 (two columns a pair): the keys stay int8 and
    // QK runs on v_mfma_i32_16x16x64_i8 against the query as an integer. Per pair, Q * scale * log2(e) is scaled
    // by 2^(22 - e) (every element then below 2^22 in magnitude, e the exponent of the pair's largest) and rounded
    // to an integer qi = 65536 L0 + 256 L1 + L2 with balanced int8 limbs (L1, L2 in [-128, 127], |L0| <= 65). The
    // pair's even column holds L0 (qb1) and L2 (qb2), its odd column L1 (qb1) and zeros (qb2), so the two columns'
    // exact int32 dot products, scaled by qcm / qc2 and added, give the score; the query is represented to 2^-23 of
    // its largest element (the f16 high/remainder split of the other kernels: 2^-22 of each element).
    constexpr bool I8M = DEC_I8_MFMA && I8 && !PM && HD != 256;
    static_assert(!I8M || NCB == 1, "the int8-MFMA QK: one column block");
    i4v qb1[HD / 64], qb2[HD / 64];
    float qcm = 0.f, qc2 = 0.f;
    {
        __amdgpu_buffer_rsrc_t rq = gi_rsrc(a.q, (long long)a.n_tok * a.q_stride * 4);
#pragma unroll
        for (int cb = 0; cb < NCB; cb++)
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                const int off = qoff[cb] + (Q4 ? 32 * kk : I8 ? 32 * (kk & 1) + 256 * (kk >> 1) : 128 * kk);
                qraw[cb][kk][0] = gi_load16(rq, off);
                qraw[cb][kk][1] = gi_load16(rq, off + 16);
            }
    }
    __builtin_amdgcn_sched_barrier(0);
    float m_run[NCB], l_run[NCB];
    // O^T: MFMA dd holds rows m = dims 8m + dd; this lane rows 4grp..4grp+3 -> dims 32grp + 8j + dd
    // (HD 256: rows m = dims 16m + dd -> dims 64grp + 16j + dd)
    f4 o[NCB][ND];
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
        m_run[cb] = GI_NEG_INF;
        l_run[cb] = 0.f;
#pragma unroll
        for (int dd = 0; dd < ND; dd++) o[cb][dd] = f4{0.f, 0.f, 0.f, 0.f};
    }

    // Loads go through buffer resources that start at the wave's current tile and end at the slice's last
    // key: offsets are 32-bit per lane, constant across tiles, and keys past the end read as zeros. DEC_NB
    // register buffers keep DEC_NB tiles in flight per wave: a buffer is refilled with the tile DEC_NB
    // ahead as soon as its data is consumed (K after the QK MFMAs, V after its transpose). Two measured
    // fastest; three or four only add register pressure.
    const long long kvs = a.kv_stride;
    const uint16_t* kslice = a.kc + (long long)k_begin * kvs + kvh * a.kv_head_stride;
    const uint16_t* vslice = a.vc + (long long)k_begin * kvs + kvh * a.kv_head_stride;
    // A-row r = c of S^T block b holds tile key 8*(c/4) + 4b + c%4; V: this lane loads keys 8grp+i, dims 8c..8c+7
    const int krow0 = 8 * (c >> 2) + (c & 3);
    const int koff0 = (krow0 * (int)kvs + 8 * grp) * 2;
    const int koff1 = koff0 + 4 * (int)kvs * 2;
    // (head size 64: V dims 4c..4c+3, so O^T block dd has rows m = dims 4m + dd)
    const int voff = (8 * grp * (int)kvs + (HD == 64 ? 4 : 8) * c) * 2;
    const int vstep = (int)kvs * 2;
    constexpr int STRIDE = WS * TILE; // keys between a wave's consecutive tiles
    // int8 element offsets (bytes): key rows of block 0 and the V rows of this lane; scales
    const int8_t* kslice8 = reinterpret_cast<const int8_t*>(a.kc) + (long long)k_begin * kvs + kvh * a.kv_head_stride;
    const int8_t* vslice8 = reinterpret_cast<const int8_t*>(a.vc) + (long long)k_begin * kvs + kvh * a.kv_head_stride;
    const long long scs = a.sc_stride;
    const float* kscl = I8 ? a.ks + (long long)k_begin * scs + kvh * a.sc_head_stride : nullptr;
    const float* vscl = I8 ? a.vs + (long long)k_begin * scs + kvh * a.sc_head_stride : nullptr;
    const int koff8 = (16 * (c >> 2) + (c & 3)) * (int)kvs + 16 * grp;
    const int voff8 = 16 * grp * (int)kvs + (HD == 64 ? 4 : 8) * c;
    const int scoff = lane * (int)scs * 4;
    // head size 256: K row c, dims 8grp + 32kk; V keys 4grp + i, dims 16c..16c+15
    const int koff256 = (c * (int)kvs + 8 * grp) * 2;
    // f16 V (DEC_V256_DENSE): the lane's two 16-byte loads of key 4grp + i are dims 8c .. 8c + 7 and 128 + 8c .. + 7, so
    // the 16 lanes of a key read two whole 256-byte runs of its row per instruction (dims 16c .. 16c + 15 put 16 bytes
    // every 32 bytes); O^T block dd then holds dims 128(dd / 8) + 8m + dd % 8 in row m
    constexpr bool V256D = DEC_V256_DENSE && HD == 256 && !I8 && !Q4;
    const int voff256 = (4 * grp * (int)kvs + (V256D ? 8 : 16) * c) * 2;
    // head size 256, int8 (byte offsets): K row c, bytes 16grp (+64i); V rows 4grp + i, bytes 16c; the scales of
    // tile key 4(lane/16) + lane%4
    const int koff256_8 = c * (int)kvs + 16 * grp;
    const int voff256_8 = 4 * grp * (int)kvs + 16 * c;
    const int scoff256 = (4 * (lane >> 4) + (lane & 3)) * (int)scs * 4;
    // 4-bit (bytes): K row c, bytes 32grp (+16); its two scales (4 bytes at f16 element 2grp of the row); V rows
    // 4grp + i, bytes 8c; their scales (f16 element c/2 of each row)
    const uint8_t* kslice4 = reinterpret_cast<const uint8_t*>(a.kc) + (long long)k_begin * kvs + kvh * a.kv_head_stride;
    const uint8_t* vslice4 = reinterpret_cast<const uint8_t*>(a.vc) + (long long)k_begin * kvs + kvh * a.kv_head_stride;
    const uint16_t* kscl4 = Q4 ? reinterpret_cast<const uint16_t*>(a.ks) + (long long)k_begin * scs + kvh * a.sc_head_stride : nullptr;
    const uint16_t* vscl4 = Q4 ? reinterpret_cast<const uint16_t*>(a.vs) + (long long)k_begin * scs + kvh * a.sc_head_stride : nullptr;
    const int koff4 = c * (int)kvs + 32 * grp;
    const int kscoff4 = (c * (int)scs + 2 * grp) * 2;
    const int voff4 = 4 * grp * (int)kvs + 8 * c;
    const int vscoff4 = (4 * grp * (int)scs + (c >> 1)) * 2;

    using Buf = typename gi_pick<Q4, DecBufQ4, DecBuf<I8, HD>>::type;
    // K/V stream loads: with WS = 4 each tile is read by one wave only, and the loads take the streaming
    // policy (at config 2 the split kernel went from 25.5 to 22.7 us with it); with WS = 2 a second wave of the
    // workgroup reads each tile again, from the caches, so the lines stay.
    constexpr int CPOL = WS == DEC_WAVES ? DEC_CPOL : 0;
    auto load_k = [&](Buf& B, int t) {
        if constexpr (Q4) {
            __amdgpu_buffer_rsrc_t r = gi_rsrc(kslice4 + (long long)t * kvs, (long long)(nkeys - t) * kvs);
            B.k[0] = gi_load16p<CPOL>(r, koff4);
            B.k[1] = gi_load16p<CPOL>(r, koff4 + 16);
            B.ksc = __builtin_amdgcn_raw_buffer_load_b32(
                gi_rsrc(kscl4 + (long long)t * scs, (long long)(nkeys - t) * scs * 2), kscoff4, 0, 0);
        } else if constexpr (HD == 256 && I8) {
            __amdgpu_buffer_rsrc_t r = gi_rsrc(kslice8 + (long long)t * kvs, (long long)(nkeys - t) * kvs);
#pragma unroll
            for (int i = 0; i < 4; i++) B.k[i] = gi_load16p<CPOL>(r, koff256_8 + 64 * i);
            B.ksc = gi_load4f(gi_rsrc(kscl + (long long)t * scs, (long long)(nkeys - t) * scs * 4), scoff256);
        } else if constexpr (HD == 256) {
            __amdgpu_buffer_rsrc_t r = gi_rsrc(kslice + (long long)t * kvs, (long long)(nkeys - t) * kvs * 2);
#pragma unroll
            for (int kk = 0; kk < 8; kk++) B.k[kk] = gi_load16p<CPOL>(r, koff256 + 64 * kk);
        } else if constexpr (I8) {
            __amdgpu_buffer_rsrc_t r = gi_rsrc(kslice8 + (long long)t * kvs, (long long)(nkeys - t) * kvs);
#pragma unroll
            for (int b = 0; b < 4; b++) {
                B.k[b][0] = gi_load16p<CPOL>(r, koff8 + 4 * b * (int)kvs);
                if constexpr (HD == 128) B.k[b][1] = gi_load16p<CPOL>(r, koff8 + 4 * b * (int)kvs + 64);
            }
            B.ksc = gi_load4f(gi_rsrc(kscl + (long long)t * scs, (long long)(nkeys - t) * scs * 4), scoff);
        } else {
            __amdgpu_buffer_rsrc_t r = gi_rsrc(kslice + (long long)t * kvs, (long long)(nkeys - t) * kvs * 2);
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                B.k[0][kk] = gi_load16p<CPOL>(r, koff0 + 64 * kk);
                B.k[1][kk] = gi_load16p<CPOL>(r, koff1 + 64 * kk);
            }
        }
    };
    auto load_v = [&](Buf& B, int t) {
        if constexpr (Q4) {
            __amdgpu_buffer_rsrc_t r = gi_rsrc(vslice4 + (long long)t * kvs, (long long)(nkeys - t) * kvs);
            __amdgpu_buffer_rsrc_t rs = gi_rsrc(vscl4 + (long long)t * scs, (long long)(nkeys - t) * scs * 2);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                B.v[i] = gi_load8p<CPOL>(r, voff4 + i * (int)kvs);
                B.vsc[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, vscoff4 + i * (int)scs * 2, 0, 0);
            }
        } else if constexpr (HD == 256 && I8) {
            __amdgpu_buffer_rsrc_t r = gi_rsrc(vslice8 + (long long)t * kvs, (long long)(nkeys - t) * kvs);
#pragma unroll
            for (int i = 0; i < 4; i++) B.v[i] = gi_load16p<CPOL>(r, voff256_8 + i * (int)kvs);
            B.vsc = gi_load4f(gi_rsrc(vscl + (long long)t * scs, (long long)(nkeys - t) * scs * 4), scoff256);
        } else if constexpr (HD == 256) {
            __amdgpu_buffer_rsrc_t r = gi_rsrc(vslice + (long long)t * kvs, (long long)(nkeys - t) * kvs * 2);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                B.v[i][0] = gi_load16p<CPOL>(r, voff256 + i * vstep);
                B.v[i][1] = gi_load16p<CPOL>(r, voff256 + i * vstep + (V256D ? 256 : 16));
            }
        } else if constexpr (I8) {
            __amdgpu_buffer_rsrc_t r = gi_rsrc(vslice8 + (long long)t * kvs, (long long)(nkeys - t) * kvs);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                if constexpr (HD == 64) B.v[i] = u2{__builtin_amdgcn_raw_buffer_load_b32(r, voff8 + i * (int)kvs, 0, CPOL), 0u};
                else B.v[i] = gi_load8p<CPOL>(r, voff8 + i * (int)kvs);
            }
            B.vsc = gi_load4f(gi_rsrc(vscl + (long long)t * scs, (long long)(nkeys - t) * scs * 4), scoff);
        } else {
            __amdgpu_buffer_rsrc_t r = gi_rsrc(vslice + (long long)t * kvs, (long long)(nkeys - t) * kvs * 2);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if constexpr (HD == 64) B.v[i] = gi_load8p<CPOL>(r, voff + i * vstep);
                else B.v[i] = gi_load16p<CPOL>(r, voff + i * vstep);
            }
        }
    };
    // One tile from buffer B at key offset t; with `reload`, B is refilled with the tile DEC_NB tiles on.
    auto process_h = [&](auto& B, int t, bool reload) {
        __builtin_amdgcn_sched_barrier(0); // keep tiles in order: each waits only for its own buffer
        f4 sacc[NCB][2];
#pragma unroll
        for (int cb = 0; cb < NCB; cb++)
#pragma unroll
            for (int b = 0; b < 2; b++) {
                sacc[cb][b] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < KK; kk++) {
                    sacc[cb][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, B.k[b][kk]), qf[cb][kk],
                                                                         sacc[cb][b], 0, 0, 0);
                    if constexpr (PM)
                        sacc[cb][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, B.k[b][kk]),
                                                                             qfl[cb][kk], sacc[cb][b], 0, 0, 0);
                }
            }
        if (reload) load_k(B, t + NB * STRIDE);
        __builtin_amdgcn_sched_barrier(0);
        const bool masked = t + DEC_TILE > span_lo; // some valid column sees only part of this tile
        h8 pf[NCB], pfl[NCB];
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
            // this lane: column c, tile keys 8grp + 4b + j
            float sc[8], mx = GI_NEG_INF;
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float v = sacc[cb][b][j];
                    if constexpr (!PM) v = v + lane_xor1(v); // hi + lo columns of the pair (same sum in both lanes)
                    sc[4 * b + j] = v;
                }
            // the mask as a real branch: only a slice's last tiles take it
            if (masked) {
                GI_KEEP_BRANCH();
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (t + 8 * grp + i >= span[cb]) sc[i] = GI_NEG_INF;
            }
#pragma unroll
            for (int i = 0; i < 8; i++) mx = fmaxf(mx, sc[i]);
            mx = rows_max(mx);
            // the column's reference max moves only when a score exceeds it by more than 2^8 in probability:
            // P <= 256 is exact enough in the f16 hi/lo split, and most tiles skip rescaling O
            const bool up = mx > m_run[cb] + DEC_RESCALE_LOG2;
            if (__builtin_amdgcn_ballot_w64(up)) {
                // alpha = 0 when nothing was seen yet; lanes that do not move keep 1 (their m_run may still be
                // -inf: a column whose keys all lie past this tile's start, beside one that sees some)
                const float m_new = up ? mx : m_run[cb];
                const float alpha = up ? __builtin_amdgcn_exp2f(m_run[cb] - m_new) : 1.f;
                m_run[cb] = m_new;
                l_run[cb] *= alpha;
#pragma unroll
                for (int dd = 0; dd < ND; dd++) gi_acc_scale<NBO == 0 && HD != 128>(o[cb][dd], alpha);
            }
            const float m_use = m_run[cb] == GI_NEG_INF ? 0.f : m_run[cb]; // no key seen yet: p = 0
            float psum = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float p = __builtin_amdgcn_exp2f(sc[i] - m_use);
                psum += p;
                _Float16 hi = (_Float16)p;
                if constexpr (PM) {
                    pf[cb][i] = hi;
                    pfl[cb][i] = (_Float16)(p - (float)hi);
                } else {
                    pf[cb][i] = (c & 1) ? (_Float16)(p - (float)hi) : hi;
                }
            }
            l_run[cb] += psum;
        }
        // O^T += V^T P^T, V^T built one dim group at a time: vt = the 8 keys' values of dim 8c + dd (head size
        // 64: 4c + dd)
#pragma unroll
        for (int dd = 0; dd < ND; dd++) {
            u4 w;
#pragma unroll
            for (int p = 0; p < 4; p++) // halves dd % 2 of keys 2p (low) and 2p + 1 (high): one v_perm
                w[p] = __builtin_amdgcn_perm(B.v[2 * p + 1][dd >> 1], B.v[2 * p][dd >> 1], (dd & 1) ? 0x07060302u : 0x05040100u);
            const h8 vt = __builtin_bit_cast(h8, w);
#pragma unroll
            for (int cb = 0; cb < NCB; cb++) {
                o[cb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vt, pf[cb], o[cb][dd], 0, 0, 0);
                if constexpr (PM) o[cb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vt, pfl[cb], o[cb][dd], 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (reload) load_v(B, t + NB * STRIDE);
    };
    // the int8 cache's QK over one 64-key tile (sacc from zero): on int8 MFMA (I8M), else the keys widened to exact f16
    auto qk_i8 = [&](auto& B, f4 (&sacc)[NCB][4]) {
        if constexpr (I8M) {
            // the key bytes as they were loaded (dims 64h + 16grp .. + 15 of the block's key), against the limbs of the
            // same dims; an exact int32 dot product per column and limb set
#pragma unroll
            for (int b = 0; b < 4; b++) {
                i4v a1 = i4v{0, 0, 0, 0}, a2 = a1;
#pragma unroll
                for (int h = 0; h < HD / 64; h++) {
                    const i4v kb = __builtin_bit_cast(i4v, B.k[b][h]);
                    a1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(kb, qb1[h], a1, 0, 0, 0);
                    a2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(kb, qb2[h], a2, 0, 0, 0);
                }
#pragma unroll
                for (int j = 0; j < 4; j++) sacc[0][b][j] = fmaf((float)a1[j], qcm, (float)a2[j] * qc2);
            }
            return;
        }
#pragma unroll
        for (int b = 0; b < 4; b++) {
            u4 kf[KK]; // k-step kk: dims 16grp + 8(kk%2) + 64(kk/2) of this block's key, as f16 pairs
#pragma unroll
            for (int half = 0; half < HD / 64; half++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t x = gi_i8_in(B.k[b][half][e]);
                    kf[2 * half + (e >> 1)][2 * (e & 1)] = i8_f16x2(x, GI_I8_LO);
                    kf[2 * half + (e >> 1)][2 * (e & 1) + 1] = i8_f16x2(x, GI_I8_HI);
                }
#pragma unroll
            for (int cb = 0; cb < NCB; cb++) {
                sacc[cb][b] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < KK; kk++) {
                    sacc[cb][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, kf[kk]), qf[cb][kk],
                                                                         sacc[cb][b], 0, 0, 0);
                    if constexpr (PM)
                        sacc[cb][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, kf[kk]), qfl[cb][kk],
                                                                             sacc[cb][b], 0, 0, 0);
                }
            }
        }
    };
    // the int8 cache's P V over one 64-key tile (pf, and with one pair per column pfl: P^T by k-step)
    auto pv_i8 = [&](auto& B, const h8 (&pf)[NCB][2], const h8 (&pfl)[NCB][2]) {
        // O^T += V^T P^T: for dims dd, dd+1 (bytes k, k+1 of word dd/4) and keys 2p, 2p+1 of a k-step, one
        // v_perm gathers the four bytes and two more widen them to the two f16 pairs
#pragma unroll
        for (int i = 0; i < 16; i++) B.v[i] = u2{gi_i8_in(B.v[i][0]), gi_i8_in(B.v[i][1])};
#pragma unroll
        for (int dd = 0; dd < ND; dd += 2) {
            const int wi = dd >> 2, k = dd & 3;
            const uint32_t sel = (uint32_t)k | (uint32_t)(k + 4) << 8 | (uint32_t)(k + 1) << 16 | (uint32_t)(k + 5) << 24;
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                u4 w0, w1;
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const uint32_t g = __builtin_amdgcn_perm(B.v[8 * ks + 2 * p + 1][wi], B.v[8 * ks + 2 * p][wi], sel);
                    w0[p] = i8_f16x2(g, GI_I8_LO);
                    w1[p] = i8_f16x2(g, GI_I8_HI);
                }
#pragma unroll
                for (int cb = 0; cb < NCB; cb++) {
                    o[cb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, w0), pf[cb][ks], o[cb][dd], 0, 0, 0);
                    o[cb][dd + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, w1), pf[cb][ks], o[cb][dd + 1], 0, 0, 0);
                    if constexpr (PM) {
                        o[cb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, w0), pfl[cb][ks], o[cb][dd], 0, 0, 0);
                        o[cb][dd + 1] =
                            __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, w1), pfl[cb][ks], o[cb][dd + 1], 0, 0, 0);
                    }
                }
            }
        }
    };
    auto process_i8 = [&](auto& B, int t, bool reload) {
        __builtin_amdgcn_sched_barrier(0);
        f4 sacc[NCB][4];
        qk_i8(B, sacc);
        const float ksc = B.ksc;
        if (reload) load_k(B, t + NB * STRIDE);
        __builtin_amdgcn_sched_barrier(0);
        // the scales of this lane's 16 keys (16grp + m, m = 4b + j)
        float ksb[16], vsb[16];
#define GI_BC(m) ksb[m] = row_bcast<m>(ksc); vsb[m] = row_bcast<m>(B.vsc);
        GI_BC(0) GI_BC(1) GI_BC(2) GI_BC(3) GI_BC(4) GI_BC(5) GI_BC(6) GI_BC(7)
        GI_BC(8) GI_BC(9) GI_BC(10) GI_BC(11) GI_BC(12) GI_BC(13) GI_BC(14) GI_BC(15)
#undef GI_BC
        const bool masked = t + TILE > span_lo;
        h8 pf[NCB][2], pfl[NCB][2]; // PV k-step ks: keys 16grp + 8ks + i
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
            float sc[16], mx = GI_NEG_INF;
#pragma unroll
            for (int m = 0; m < 16; m++) {
                float v = sacc[cb][m >> 2][m & 3];
                if constexpr (!PM) v = v + lane_xor1(v); // hi + lo columns of the pair
                v *= ksb[m];                             // the key's scale
                sc[m] = v;
            }
            // the mask as a real branch, which only a slice's last tiles take (int8 decode measured 2% faster
            // than with the selects on every tile; the f16 kernels gain nothing)
            if (masked) {
                GI_KEEP_BRANCH();
#pragma unroll
                for (int m = 0; m < 16; m++)
                    if (t + 16 * grp + m >= span[cb]) sc[m] = GI_NEG_INF;
            }
#pragma unroll
            for (int m = 0; m < 16; m++) mx = fmaxf(mx, sc[m]);
            mx = rows_max(mx);
            const bool up = mx > m_run[cb] + DEC_RESCALE_LOG2;
            if (__builtin_amdgcn_ballot_w64(up)) {
                const float m_new = up ? mx : m_run[cb];
                const float alpha = up ? __builtin_amdgcn_exp2f(m_run[cb] - m_new) : 1.f;
                m_run[cb] = m_new;
                l_run[cb] *= alpha;
#pragma unroll
                for (int dd = 0; dd < ND; dd++) gi_acc_scale<NBO == 0 && HD != 128>(o[cb][dd], alpha);
            }
            const float m_use = m_run[cb] == GI_NEG_INF ? 0.f : m_run[cb];
            float psum = 0.f;
#pragma unroll
            for (int m = 0; m < 16; m++) {
                const float p = __builtin_amdgcn_exp2f(sc[m] - m_use);
                psum += p;
                const float pv = p * vsb[m] * (PM ? DEC_I8_VB : 1.f);
                _Float16 hi = (_Float16)pv;
                if constexpr (PM) {
                    pf[cb][m >> 3][m & 7] = hi;
                    pfl[cb][m >> 3][m & 7] = (_Float16)(pv - (float)hi);
                } else {
                    pf[cb][m >> 3][m & 7] = (c & 1) ? (_Float16)((pv - (float)hi) * DEC_I8_LO) : hi;
                }
            }
            l_run[cb] += psum;
        }
        pv_i8(B, pf, pfl);
        __builtin_amdgcn_sched_barrier(0);
        if (reload) load_v(B, t + NB * STRIDE);
    };
    // K fragment of k-step kk of a head-size-256 tile (int8: the lane's 8 bytes of dims 64(kk/2) + 16grp +
    // 8(kk%2), widened; 4-bit: its values 64grp + 8kk .. + 7, widened with their scale)
    auto kfrag256 = [&](auto& B, int kk) -> h8 {
        if constexpr (Q4) {
            // values 64grp + 8kk .. + 7: bytes 4kk .. 4kk + 3 of the lane's 32, scale group 2grp + kk/4
            const uint32_t x = B.k[kk >> 2][kk & 3];
            const h2x sc = __builtin_bit_cast(h2x, (kk >> 2) ? (B.ksc >> 16) * 0x10001u : (B.ksc & 0xffffu) * 0x10001u);
            const uint32_t hi = x >> 4;
            return __builtin_bit_cast(h8, u4{q4_f16x2(hi, x, 0, sc), q4_f16x2(hi, x, 1, sc), q4_f16x2(hi, x, 2, sc),
                                             q4_f16x2(hi, x, 3, sc)});
        } else if constexpr (I8) {
            const uint32_t x0 = gi_i8_in(B.k[kk >> 1][2 * (kk & 1)]), x1 = gi_i8_in(B.k[kk >> 1][2 * (kk & 1) + 1]);
            return __builtin_bit_cast(h8, u4{i8_f16x2(x0, GI_I8_LO), i8_f16x2(x0, GI_I8_HI), i8_f16x2(x1, GI_I8_LO),
                                             i8_f16x2(x1, GI_I8_HI)});
        } else {
            return __builtin_bit_cast(h8, B.k[kk]);
        }
    };
    // O^T += V^T P^T over a head-size-256 tile (P^T: the high parts pf and, with one pair per column, the
    // remainders pfl)
    auto pv256 = [&](auto& B, const h4x (&pf)[NCB], const h4x (&pfl)[NCB]) {
        // V^T block dd: element i of the A operand = V[key 4grp + i][dim 16c + dd]. int8: for dims dd, dd + 1
        // and keys 2p, 2p + 1 one v_perm gathers the four bytes and two converts widen them to f16 pairs
        u2 v8[16];
        if constexpr (I8) {
#pragma unroll
            for (int dd = 0; dd < 16; dd += 2) {
                const int wi = dd >> 2, k = dd & 3;
                const uint32_t sel = (uint32_t)k | (uint32_t)(k + 4) << 8 | (uint32_t)(k + 1) << 16 | (uint32_t)(k + 5) << 24;
#pragma unroll
                for (int p = 0; p < 2; p++) {
                    const uint32_t g = __builtin_amdgcn_perm(gi_i8_in(B.v[2 * p + 1][wi]), gi_i8_in(B.v[2 * p][wi]), sel);
                    v8[dd][p] = i8_f16x2(g, GI_I8_LO);
                    v8[dd + 1][p] = i8_f16x2(g, GI_I8_HI);
                }
            }
        }
        // 4-bit: for keys 2p, 2p + 1 the pair (key 2p, key 2p + 1) of dim 16c + dd is nibble dd%2 of byte dd/2 of
        // each row, each times its own key's scale
        h2x vsp[2];
        if constexpr (Q4) {
#pragma unroll
            for (int p = 0; p < 2; p++)
                vsp[p] = __builtin_bit_cast(h2x, (B.vsc[2 * p] & 0xffffu) | (B.vsc[2 * p + 1] << 16));
        }
#pragma unroll
        for (int dd = 0; dd < 16; dd++) {
            u2 vw;
            if constexpr (Q4) {
                const int w = dd >> 3, j = (dd >> 1) & 3;
#pragma unroll
                for (int p = 0; p < 2; p++) {
                    const uint32_t xa = B.v[2 * p][w], xb = B.v[2 * p + 1][w];
                    vw[p] = (dd & 1) ? q4_f16x2(xb >> 4, xa >> 4, j, vsp[p]) : q4_f16x2(xb, xa, j, vsp[p]);
                }
            } else if constexpr (I8) {
                vw = v8[dd];
            } else {
                const int h = dd >> 3, w = (dd & 7) >> 1;
#pragma unroll
                for (int p = 0; p < 2; p++)
                    vw[p] = __builtin_amdgcn_perm(B.v[2 * p + 1][h][w], B.v[2 * p][h][w], (dd & 1) ? 0x07060302u : 0x05040100u);
            }
            const h4x vt = __builtin_bit_cast(h4x, vw);
#pragma unroll
            for (int cb = 0; cb < NCB; cb++) {
                o[cb][dd] = __builtin_amdgcn_mfma_f32_16x16x16f16(vt, pf[cb], o[cb][dd], 0, 0, 0);
                if constexpr (PM && !REF) o[cb][dd] = __builtin_amdgcn_mfma_f32_16x16x16f16(vt, pfl[cb], o[cb][dd], 0, 0, 0);
            }
        }
    };
    auto process_256 = [&](auto& B, int t, bool reload) {
        __builtin_amdgcn_sched_barrier(0);
        f4 sacc[NCB];
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) sacc[cb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            const h8 kf = kfrag256(B, kk);
#pragma unroll
            for (int cb = 0; cb < NCB; cb++) {
                sacc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[cb][kk], sacc[cb], 0, 0, 0);
                if constexpr (PM && !REF) sacc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qfl[cb][kk], sacc[cb], 0, 0, 0);
            }
        }
        float ksb[4], vsb[4]; // int8: the scales of keys 4grp + j
        if constexpr (I8) {
            ksb[0] = row_bcast<0>(B.ksc), ksb[1] = row_bcast<1>(B.ksc), ksb[2] = row_bcast<2>(B.ksc), ksb[3] = row_bcast<3>(B.ksc);
            vsb[0] = row_bcast<0>(B.vsc), vsb[1] = row_bcast<1>(B.vsc), vsb[2] = row_bcast<2>(B.vsc), vsb[3] = row_bcast<3>(B.vsc);
        }
        if (reload) load_k(B, t + NB * STRIDE);
        __builtin_amdgcn_sched_barrier(0);
        const bool masked = t + TILE > span_lo;
        h4x pf[NCB], pfl[NCB]; // PV B operand: keys 4grp + j of column c (PM: high parts and remainders)
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
            float sc[4], mx = GI_NEG_INF;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float v = sacc[cb][j];
                if constexpr (!PM) v = v + lane_xor1(v); // hi + lo columns of the pair
                if constexpr (I8) v *= ksb[j];           // the key's scale
                sc[j] = v;
            }
            if (masked) {
                GI_KEEP_BRANCH();
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (t + 4 * grp + j >= span[cb]) sc[j] = GI_NEG_INF;
            }
#pragma unroll
            for (int j = 0; j < 4; j++) mx = fmaxf(mx, sc[j]);
            mx = rows_max(mx);
            const bool up = mx > m_run[cb] + DEC_RESCALE_LOG2;
            if (__builtin_amdgcn_ballot_w64(up)) {
                const float m_new = up ? mx : m_run[cb];
                const float alpha = up ? __builtin_amdgcn_exp2f(m_run[cb] - m_new) : 1.f;
                m_run[cb] = m_new;
                l_run[cb] *= alpha;
#pragma unroll
                for (int dd = 0; dd < ND; dd++) gi_acc_scale<NBO == 0 && HD != 128>(o[cb][dd], alpha);
            }
            const float m_use = m_run[cb] == GI_NEG_INF ? 0.f : m_run[cb];
            float psum = 0.f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float p = __builtin_amdgcn_exp2f(sc[j] - m_use);
                psum += p;
                // int8: P V takes p times the value's scale (biased like the head-128 int8 kernel)
                const float pv = I8 ? p * vsb[j] * PBIAS : p;
                _Float16 hi = (_Float16)pv;
                if constexpr (REF) {
                    pf[cb][j] = hi; // rounded once, as the reference's pack_h2 (src/cuda.rs:2723)
                } else if constexpr (PM) {
                    pf[cb][j] = hi;
                    pfl[cb][j] = (_Float16)(pv - (float)hi);
                } else {
                    pf[cb][j] = (c & 1) ? (_Float16)((pv - (float)hi) * (I8 ? DEC_I8_LO : 1.f)) : hi;
                }
            }
            l_run[cb] += psum;
        }
        pv256(B, pf, pfl);
        __builtin_amdgcn_sched_barrier(0);
        if (reload) load_v(B, t + NB * STRIDE);
    };
    // ---- software pipeline of the one-pair-per-column kernels over the f16 and 4-bit caches: a tile's QK runs one
    // step ahead, so the MFMAs of tile t+1's QK interleave with tile t's exp and packing, and tile t's PV MFMAs
    // with tile t+1's row max. Unmasked tiles only; the rest take process_h / process_256. Scores come out of the
    // MFMA relative to the column's reference max (each chain starts from C = -max), so the exp takes them as
    // they are; a tile that moves the reference shifts its own scores by the change.
    // int8 (head size 128): the key scales multiply the MFMA's dot products, so the scores are made relative
    // (s * kscale - max) in one FMA each before the row max, and P V takes p times the value scale.
    constexpr int PB = HD == 256 ? 1 : I8 ? 4 : 2;              // S^T blocks of 16 keys per column block
    typedef typename gi_pick<HD == 256, h4x, h8>::type PT;     // PV B operand: 16 or 32 keys of one column
    typedef typename gi_pick<I8 && HD != 256, PT[2], PT>::type PE; // a column's P^T for the tile (int8: 2 k-steps)
    struct PipeS { f4 v[NCB][PB]; float ksc; };
    struct PipeP { PE hi[NCB], lo[NCB]; };
    auto pm_qk = [&](auto& B, PipeS& S) {
        if constexpr (I8 && HD != 256) {
            f4 sacc[NCB][4];
            qk_i8(B, sacc);
#pragma unroll
            for (int cb = 0; cb < NCB; cb++)
#pragma unroll
                for (int b = 0; b < PB; b++) {
                    asm volatile("" : "+v"(sacc[cb][b]));
                    S.v[cb][b] = sacc[cb][b];
                }
            S.ksc = B.ksc; // (the K buffer is refilled before this tile's max)
            return;
        }
        if constexpr (I8) S.ksc = B.ksc;
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
            // int8: the chains start from zero (the key scales come after the dot products)
            const float mu = I8 || m_run[cb] == GI_NEG_INF ? 0.f : m_run[cb];
#pragma unroll
            for (int b = 0; b < PB; b++) {
                f4 acc = f4{-mu, -mu, -mu, -mu};
#pragma unroll
                for (int kk = 0; kk < KK; kk++) {
                    h8 kf;
                    if constexpr (HD == 256) kf = kfrag256(B, kk);
                    else kf = __builtin_bit_cast(h8, B.k[b][kk]);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[cb][kk], acc, 0, 0, 0);
                    if constexpr (!REF) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qfl[cb][kk], acc, 0, 0, 0);
                }
                // (in VGPRs once, for the max and then the exp, instead of two reads of an accumulator register)
                asm volatile("" : "+v"(acc));
                S.v[cb][b] = acc;
            }
        }
    };
    // the tile's row max per column, and the lazy rescale of O when the reference moves (by more than 2^8; the
    // first tile sets it), which also shifts the tile's scores onto the new reference
    auto pm_max = [&](PipeS& S) {
        float mx[NCB];
        bool up[NCB];
        bool any = false;
        if constexpr (I8) {
            // the scales of this lane's keys (head size 128: 16grp + m, m = 4b + j; 256: 4grp + m), and the scores
            // relative to the reference
            float ksb[4 * PB];
#define GI_BC(m) ksb[m] = row_bcast<m>(S.ksc);
            GI_BC(0) GI_BC(1) GI_BC(2) GI_BC(3)
            if constexpr (PB == 4) { GI_BC(4) GI_BC(5) GI_BC(6) GI_BC(7) GI_BC(8) GI_BC(9) GI_BC(10) GI_BC(11)
                                     GI_BC(12) GI_BC(13) GI_BC(14) GI_BC(15) }
#undef GI_BC
#pragma unroll
            for (int cb = 0; cb < NCB; cb++) {
                const float mu = m_run[cb] == GI_NEG_INF ? 0.f : m_run[cb];
#pragma unroll
                for (int m = 0; m < 4 * PB; m++) S.v[cb][m >> 2][m & 3] = fmaf(S.v[cb][m >> 2][m & 3], ksb[m], -mu);
            }
        }
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
            // a chain of three-input maxima over the column's 4 PB scores
            float m = fmaxf(fmaxf(S.v[cb][0][0], S.v[cb][0][1]), S.v[cb][0][2]);
#pragma unroll
            for (int k = 3; k + 1 < 4 * PB; k += 2)
                m = fmaxf(fmaxf(m, S.v[cb][k >> 2][k & 3]), S.v[cb][(k + 1) >> 2][(k + 1) & 3]);
            if constexpr ((4 * PB - 3) % 2 == 1) m = fmaxf(m, S.v[cb][PB - 1][3]);
            mx[cb] = rows_max(m);
            up[cb] = m_run[cb] == GI_NEG_INF || mx[cb] > DEC_RESCALE_LOG2;
            any = any || up[cb];
        }
        if (__builtin_amdgcn_ballot_w64(any)) {
#pragma unroll
            for (int cb = 0; cb < NCB; cb++) {
                const float mu = m_run[cb] == GI_NEG_INF ? 0.f : m_run[cb];
                const float m_new = up[cb] ? mx[cb] + mu : m_run[cb];
                const float alpha = up[cb] ? __builtin_amdgcn_exp2f(m_run[cb] - m_new) : 1.f;
                const float delta = up[cb] ? m_new - mu : 0.f;
                m_run[cb] = m_new;
                l_run[cb] *= alpha;
#pragma unroll
                for (int dd = 0; dd < ND; dd++) gi_acc_scale<NBO == 0 && HD != 128>(o[cb][dd], alpha);
#pragma unroll
                for (int b = 0; b < PB; b++) S.v[cb][b] -= delta;
            }
        }
    };
    auto pm_exp = [&](auto& B, const PipeS& S, PipeP& P) {
        float vsb[4 * PB]; // int8: the value scales of this lane's keys
        if constexpr (I8) {
#define GI_BC(m) vsb[m] = row_bcast<m>(B.vsc);
            GI_BC(0) GI_BC(1) GI_BC(2) GI_BC(3)
            if constexpr (PB == 4) { GI_BC(4) GI_BC(5) GI_BC(6) GI_BC(7) GI_BC(8) GI_BC(9) GI_BC(10) GI_BC(11)
                                     GI_BC(12) GI_BC(13) GI_BC(14) GI_BC(15) }
#undef GI_BC
        }
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
            float psum = 0.f;
#pragma unroll
            for (int i = 0; i < 4 * PB; i++) {
                const float p = __builtin_amdgcn_exp2f(S.v[cb][i >> 2][i & 3]);
                psum += p;
                // int8: P V takes p times the value's scale (biased like process_i8)
                const float pv = I8 ? p * vsb[i] * PBIAS : p;
                // the high part: pv cut to f16's 11 significant bits, so that it converts exactly and the
                // remainder is an exact f32 subtraction (no conversion back)
                const float hi = __uint_as_float(__float_as_uint(pv) & 0xffffe000u);
                if constexpr (REF) {
                    P.hi[cb][i] = (_Float16)pv; // rounded once, as the reference's pack_h2 (src/cuda.rs:2723)
                } else if constexpr (I8 && HD != 256) {
                    P.hi[cb][i >> 3][i & 7] = (_Float16)hi;
                    P.lo[cb][i >> 3][i & 7] = (_Float16)(pv - hi);
                } else {
                    P.hi[cb][i] = (_Float16)hi;
                    P.lo[cb][i] = (_Float16)(pv - hi);
                }
            }
            l_run[cb] += psum;
        }
    };
    auto pm_pv = [&](auto& B, const PipeP& P) {
        if constexpr (HD == 256) {
            pv256(B, P.hi, P.lo);
        } else if constexpr (I8) {
            pv_i8(B, P.hi, P.lo);
        } else {
#pragma unroll
            for (int dd = 0; dd < ND; dd++) {
                u4 w;
#pragma unroll
                for (int p = 0; p < 4; p++)
                    w[p] = __builtin_amdgcn_perm(B.v[2 * p + 1][dd >> 1], B.v[2 * p][dd >> 1],
                                                 (dd & 1) ? 0x07060302u : 0x05040100u);
                const h8 vt = __builtin_bit_cast(h8, w);
#pragma unroll
                for (int cb = 0; cb < NCB; cb++) {
                    o[cb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vt, P.hi[cb], o[cb][dd], 0, 0, 0);
                    o[cb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vt, P.lo[cb], o[cb][dd], 0, 0, 0);
                }
            }
        }
    };
    auto process = [&](Buf& B, int t, bool reload) {
        if constexpr (HD == 256) process_256(B, t, reload);
        else if constexpr (I8) process_i8(B, t, reload);
        else process_h(B, t, reload);
    };

    // (the first loads are issued unconditionally, before the loop, so every iteration starts with the same
    // loads outstanding and the compiler's load counters wait for exactly the buffer in use)
    // a pair set whose pairs all lie past the last one has nothing to compute (its waves still join the merge)
    if (pair0 < npairs) {
    Buf B[NB];
    const int t_first = (wave % WS) * TILE;
    // Only the first tile is requested before the queries are converted; the other buffers are requested once
    // its keys have arrived. The launch's first requests are then a smaller burst, which the memory system
    // serves sooner, and the first tile's arithmetic starts earlier (measured faster for every kernel but the
    // f16 one-pair-per-column ones, whose pipelined loop wants every buffer from the start).
    constexpr bool DEFER = !PM || I8 || Q4;
#pragma unroll
    for (int i = 0; i < (DEFER ? 1 : NB); i++) {
        load_k(B[i], t_first + i * STRIDE);
        __builtin_amdgcn_sched_barrier(0);
        load_v(B[i], t_first + i * STRIDE);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (I8M) {
        float qv[KK][8];
        float mx = 0.f;
#pragma unroll
        for (int kk = 0; kk < KK; kk++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t bits = qraw[0][kk][e >> 2][e & 3];
                qv[kk][e] = valid[0] ? __uint_as_float(bits) * a.qscale : 0.f;
                mx = fmaxf(mx, fabsf(qv[kk][e]));
            }
        // the pair's row spans the lanes c, c + 16, c + 32, c + 48
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const int ex = mx > 0.f ? __builtin_amdgcn_frexp_expf(mx) : 0; // mx < 2^ex
        const float up = __builtin_ldexpf(1.f, 22 - ex);
        qc2 = __builtin_ldexpf(1.f, ex - 22);
        qcm = __builtin_ldexpf(1.f, ex - ((c & 1) ? 14 : 6));
#pragma unroll
        for (int h = 0; h < HD / 64; h++) {
            uint32_t w1[4], w2[4];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                w1[w] = 0u;
                w2[w] = 0u;
            }
#pragma unroll
            for (int j = 0; j < 16; j++) {
                // element j of the lane's 16 dims of this half: k-step 2h + j / 8, element j % 8
                const int qi = __float2int_rn(qv[2 * h + (j >> 3)][j & 7] * up);
                const int l2 = ((qi + 128) & 255) - 128;
                const int q1 = (qi - l2) >> 8;
                const int l1 = ((q1 + 128) & 255) - 128;
                const int l0 = (q1 - l1) >> 8;
                const uint32_t b1 = (uint32_t)((c & 1) ? l1 : l0) & 255u, b2 = (c & 1) ? 0u : (uint32_t)l2 & 255u;
                w1[j >> 2] |= b1 << (8 * (j & 3));
                w2[j >> 2] |= b2 << (8 * (j & 3));
            }
            qb1[h] = i4v{(int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3]};
            qb2[h] = i4v{(int)w2[0], (int)w2[1], (int)w2[2], (int)w2[3]};
        }
    } else
    // Q * scale * log2(e) in f32, split into an f16 high part (even columns) and its f16 remainder (odd)
#pragma unroll
    for (int cb = 0; cb < NCB; cb++)
#pragma unroll
        for (int kk = 0; kk < KK; kk++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                // (the element is copied to a scalar first: clang's __builtin_bit_cast of a vector-element
                // lvalue reads element 0)
                const uint32_t bits = qraw[cb][kk][e >> 2][e & 3];
                float v = valid[cb] ? __uint_as_float(bits) * a.qscale : 0.f;
                _Float16 hi = (_Float16)v;
                if constexpr (REF) {
                    qf[cb][kk][e] = hi; // rounded once, as the reference's qf (src/cuda.rs:2669)
                } else if constexpr (PM) {
                    qf[cb][kk][e] = hi;
                    qfl[cb][kk][e] = (_Float16)(v - (float)hi);
                } else {
                    qf[cb][kk][e] = (c & 1) ? (_Float16)(v - (float)hi) : hi;
                }
            }
    if constexpr (DEFER) {
        gi_touch(B[0].k);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 1; i < NB; i++) {
            load_k(B[i], t_first + i * STRIDE);
            __builtin_amdgcn_sched_barrier(0);
            load_v(B[i], t_first + i * STRIDE);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // Steady state: every buffer gets a further tile (those past the slice read zeros and are never
    // processed). The last round of tiles runs without reloads, so no load is left in flight at the end.
    int t = t_first;
    if constexpr (DEC_PIPE && PM && NB % 2 == 0) { // (its two score sets alternate with the buffers: NB even)
        // State at the top of each step: tile t in B[0] with its scores (row max taken, O rescaled), its K buffer
        // already refilled with tile t + NB STRIDE; tiles t + i STRIDE in B[i]. A step finishes tiles t ..
        // t + (NB-1) STRIDE and scores tile t + NB STRIDE, so it runs while that tile needs no mask.
        if (t + NB * STRIDE + TILE <= span_lo) {
            PipeS S[2];
            PipeP P;
            pm_qk(B[0], S[0]);
            load_k(B[0], t + NB * STRIDE);
            pm_max(S[0]);
            do {
#pragma unroll
                for (int i = 0; i < NB; i++) {
                    __builtin_amdgcn_sched_barrier(0);
                    pm_qk(B[(i + 1) % NB], S[(i + 1) & 1]);
                    pm_exp(B[i], S[i & 1], P);
                    load_k(B[(i + 1) % NB], t + (i + 1 + NB) * STRIDE);
                    pm_pv(B[i], P);
                    pm_max(S[(i + 1) & 1]);
                    load_v(B[i], t + (i + NB) * STRIDE);
                }
                t += NB * STRIDE;
            } while (t + NB * STRIDE + TILE <= span_lo);
            __builtin_amdgcn_sched_barrier(0);
            // finish tile t; B[0] then holds tile t + NB STRIDE and B[i] tile t + i STRIDE, which the per-tile path
            // takes, so the steps below start from t + NB STRIDE with the buffers in order
            pm_exp(B[0], S[0], P);
            pm_pv(B[0], P);
            load_v(B[0], t + NB * STRIDE);
#pragma unroll
            for (int i = 1; i < NB; i++)
                if (t + i * STRIDE < nkeys) process(B[i], t + i * STRIDE, true);
            t += NB * STRIDE;
        }
    }
    for (; t + NB * STRIDE < nkeys; t += NB * STRIDE) {
#pragma unroll
        for (int i = 0; i < NB; i++) process(B[i], t + i * STRIDE, true);
    }
#pragma unroll
    for (int i = 0; i < NB; i++)
        if (t + i * STRIDE < nkeys) process(B[i], t + i * STRIDE, false);
    }

    // ---- wave results to LDS: every lane's 32 O^T values (its column, dims 32grp + 8j + dd) as 8 16-byte
    // stores; per pair the max and the sum over the 4 k-groups
    // (HD 256: 64 values, dims 64grp + 16j + dd, as 16 stores)
    __shared__ __attribute__((aligned(16))) float sm_o[DEC_WAVES][16 * NCB][HD + 4];
    __shared__ float sm_m[DEC_WAVES][CPAIRS * NCB], sm_l[DEC_WAVES][CPAIRS * NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
        float l = rows_sum(l_run[cb]);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // (V256D: row m = 4grp + j of block dd is dim 128(dd / 8) + 8m + dd % 8)
            float* row = &sm_o[wave][16 * cb + c][V256D ? 8 * (4 * grp + j) : (HD / 4) * grp + (ND)*j];
#pragma unroll
            for (int q4 = 0; q4 < ND / 4; q4++)
                *reinterpret_cast<float4*>(row + (V256D ? 128 * (q4 >> 1) + 4 * (q4 & 1) : 4 * q4)) =
                    make_float4(o[cb][4 * q4][j], o[cb][4 * q4 + 1][j], o[cb][4 * q4 + 2][j], o[cb][4 * q4 + 3][j]);
        }
        if (lane < 16 && (PM || (c & 1) == 0)) {
            sm_m[wave][cb * CPAIRS + (PM ? c : c >> 1)] = m_run[cb];
            sm_l[wave][cb * CPAIRS + (PM ? c : c >> 1)] = l;
        }
    }
    __syncthreads();
    // ---- merge each pair set's waves and the hi/lo columns: thread -> (pair, 4 dims)
    constexpr float LO = I8 ? 1.f / DEC_I8_LO : 1.f;      // the remainder column's scale (PM: no column)
    constexpr float OSC = 1.f / PBIAS; // the bias on P (int8 with one pair per column)
    // all LDS reads of the thread's items are issued before any arithmetic, so the merge waits for LDS once
    // (head size 64 with 8 pairs: 128 items, so threads 128-255 have none)
    constexpr int NITEM = WG_PAIRS * HD / 4, ITEMS = (NITEM + 255) / 256;
    float mw[ITEMS][WS], lw[ITEMS][WS];
    float4 ohi[ITEMS][WS], olo[ITEMS][WS];
#pragma unroll
    for (int it = 0; it < ITEMS; it++) {
        const int item = threadIdx.x + 256 * it;
        if (NITEM % 256 && item >= NITEM) break;
        const int pl = item / (HD / 4), d4 = 4 * (item % (HD / 4)); // pair within the workgroup
        const int w0 = (pl / (CPAIRS * NCB)) * WS;                    // the waves holding the pair
        const int lp = pl % (CPAIRS * NCB);                            // the pair within those waves
        const int row = PM ? lp : 16 * (lp >> 3) + 2 * (lp & 7);       // its (first) column
#pragma unroll
        for (int w = 0; w < WS; w++) {
            mw[it][w] = sm_m[w0 + w][lp];
            lw[it][w] = sm_l[w0 + w][lp];
            ohi[it][w] = *reinterpret_cast<const float4*>(&sm_o[w0 + w][row][d4]);
            if constexpr (!PM) olo[it][w] = *reinterpret_cast<const float4*>(&sm_o[w0 + w][row + 1][d4]);
        }
    }
#pragma unroll
    for (int it = 0; it < ITEMS; it++) {
        const int item = threadIdx.x + 256 * it;
        if (NITEM % 256 && item >= NITEM) break;
        const int pl = item / (HD / 4), d4 = 4 * (item % (HD / 4));
        const int pi = gz * WG_PAIRS + pl;
        float M = GI_NEG_INF;
#pragma unroll
        for (int w = 0; w < WS; w++) M = fmaxf(M, mw[it][w]);
        float L = 0.f;
        float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
        if (M != GI_NEG_INF) {
#pragma unroll
            for (int w = 0; w < WS; w++) {
                const float wt = __builtin_amdgcn_exp2f(mw[it][w] - M);
                L += wt * lw[it][w];
                const float4 hi = ohi[it][w];
                if constexpr (PM) {
                    const float ws = wt * OSC;
                    O.x += ws * hi.x;
                    O.y += ws * hi.y;
                    O.z += ws * hi.z;
                    O.w += ws * hi.w;
                } else {
                    const float4 lo = olo[it][w];
                    O.x += wt * (hi.x + lo.x * LO);
                    O.y += wt * (hi.y + lo.y * LO);
                    O.z += wt * (hi.z + lo.z * LO);
                    O.w += wt * (hi.w + lo.w * LO);
                }
            }
        }
        if (pi < npairs) {
            const int tk = pi / G, h = kvh * G + pi % G;
            if (a.nsplit == 1) {
                const float inv = 1.f / L;
                *reinterpret_cast<float4*>(a.out + (long long)tk * a.out_stride + (long long)h * HD + d4) =
                    make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
            } else {
                float* p = a.part + (((long long)tk * a.n_heads + h) * a.nsplit + s) * PART;
                *reinterpret_cast<float4*>(p + d4) = O;
                if (d4 == 0) *reinterpret_cast<float2*>(p + HD) = make_float2(M, L);
            }
        }
    }
}

#define GI_DEC_KERNEL(name, NCB, WS, I8, HD) \
    extern "C" __global__ void __launch_bounds__(256, DEC_MINWG) name(GiDecodeArgs a) { gi_decode_partial_t<NCB, WS, I8, HD>(a); }
#define GI_DEC_PM_KERNEL(name, NCB, WS, I8) \
    extern "C" __global__ void __launch_bounds__(256, DEC_MINWG) name(GiDecodeArgs a) { gi_decode_partial_t<NCB, WS, I8, 128, true>(a); }
GI_DEC_KERNEL(gi_decode_partial_1, 1, DEC_WAVES, false, 128)
// Short spans (at most two tiles per wave, as at config 1's 4096 keys): one register buffer, and the register budget of
// two workgroups per CU, 161 registers against 264. Config 1, graph-replayed step, two alternating runs on one box: 8.95 /
// 8.95 µs against 9.47 / 9.46 with the default kernel; at config 2 the same build measured level with it.
extern "C" __global__ void __launch_bounds__(256, 2) gi_decode_partial_1s(GiDecodeArgs a) {
    gi_decode_partial_t<1, DEC_WAVES, false, 128, false, false, false, 1>(a);
}
// the same over the int8 cache (tiles of 64 keys) and at head size 64
extern "C" __global__ void __launch_bounds__(256, 2) gi_decode_partial_1s_i8(GiDecodeArgs a) {
    gi_decode_partial_t<1, DEC_WAVES, true, 128, false, false, false, 1>(a);
}
extern "C" __global__ void __launch_bounds__(256, 2) gi_decode_partial_1s_h64(GiDecodeArgs a) {
    gi_decode_partial_t<1, DEC_WAVES, false, 64, false, false, false, 1>(a);
}
// head size 256 (16-key tiles): the f16 cache, and the int8 and 4-bit caches' tc256 kernels (which otherwise keep four
// tiles in flight)
extern "C" __global__ void __launch_bounds__(256, 2) gi_decode_partial_1s_h256(GiDecodeArgs a) {
    gi_decode_partial_t<1, DEC_WAVES, false, 256, false, false, false, 1>(a);
}
extern "C" __global__ void __launch_bounds__(256, 2) gi_decode_pm_1s_i8_h256(GiDecodeArgs a) {
    gi_decode_partial_t<1, DEC_WAVES, true, 256, true, false, false, 1>(a);
}
extern "C" __global__ void __launch_bounds__(256, 2) gi_decode_pm_1s_q4(GiDecodeArgs a) {
    gi_decode_partial_t<1, DEC_WAVES, false, 256, true, true, false, 1>(a);
}
// head size 64 (the reference's attention_partial_gqa at any head size a multiple of 32, src/cuda.rs:1684-1865)
#define GI_DEC_PM64_KERNEL(name, NCB, I8) \
    extern "C" __global__ void __launch_bounds__(256, DEC_MINWG) name(GiDecodeArgs a) { gi_decode_partial_t<NCB, DEC_WAVES, I8, 64, true>(a); }
GI_DEC_KERNEL(gi_decode_partial_1_h64, 1, DEC_WAVES, false, 64)
GI_DEC_KERNEL(gi_decode_partial_1_i8_h64, 1, DEC_WAVES, true, 64)
GI_DEC_PM64_KERNEL(gi_decode_pm_1_h64, 1, false)
GI_DEC_PM64_KERNEL(gi_decode_pm_2_h64, 2, false)
GI_DEC_PM64_KERNEL(gi_decode_pm_1_i8_h64, 1, true)
GI_DEC_PM64_KERNEL(gi_decode_pm_2_i8_h64, 2, true)
GI_DEC_KERNEL(gi_decode_partial_1_i8, 1, DEC_WAVES, true, 128)
GI_DEC_KERNEL(gi_decode_partial_1_h256, 1, DEC_WAVES, false, 256)
GI_DEC_PM_KERNEL(gi_decode_pm_1, 1, DEC_WAVES, false)
GI_DEC_PM_KERNEL(gi_decode_pm_2, 2, DEC_WAVES, false)
GI_DEC_PM_KERNEL(gi_decode_pm_1_i8, 1, DEC_WAVES, true)
GI_DEC_PM_KERNEL(gi_decode_pm_2_i8, 2, DEC_WAVES, true)
GI_DEC_PM_KERNEL(gi_decode_pm_ws2_2, 2, 2, false)
GI_DEC_PM_KERNEL(gi_decode_pm_ws2_2_i8, 2, 2, true)
#define GI_DEC_PM256_KERNEL(name, NCB, WS, I8) \
    extern "C" __global__ void __launch_bounds__(256, DEC_MINWG) name(GiDecodeArgs a) { gi_decode_partial_t<NCB, WS, I8, 256, true>(a); }
#define GI_DEC_Q4_KERNEL(name, NCB, WS) \
    extern "C" __global__ void __launch_bounds__(256, DEC_MINWG) name(GiDecodeArgs a) { gi_decode_partial_t<NCB, WS, false, 256, true, true>(a); }
GI_DEC_PM256_KERNEL(gi_decode_pm_ws2_1_h256, 1, 2, false)
// head size 256 over the int8 and 4-bit caches: the reference's tc256 roundings, 16 pairs per workgroup, or 32 as
// two pair sets (int8) or two column blocks per wave (4-bit)
GI_DEC_PM256_KERNEL(gi_decode_pm_1_i8_h256, 1, DEC_WAVES, true)
GI_DEC_PM256_KERNEL(gi_decode_pm_ws2_1_i8_h256, 1, 2, true)
GI_DEC_Q4_KERNEL(gi_decode_pm_1_q4, 1, DEC_WAVES)
GI_DEC_Q4_KERNEL(gi_decode_pm_2_q4, 2, DEC_WAVES)
// head size 256 over the int8 cache in f32 precision (the f16 cache's layouts: up to 8 pairs the high/remainder
// columns, above two pair sets of 16 per workgroup)
extern "C" __global__ void __launch_bounds__(256, DEC_MINWG) gi_decode_partial_1_i8_h256f(GiDecodeArgs a) {
    gi_decode_partial_t<1, DEC_WAVES, true, 256, false, false, true>(a);
}
extern "C" __global__ void __launch_bounds__(256, DEC_MINWG) gi_decode_pm_ws2_1_i8_h256f(GiDecodeArgs a) {
    gi_decode_partial_t<1, 2, true, 256, true, false, true>(a);
}


// Merge the slices of each (token, head): M = max m_s, w_s = 2^(m_s - M), out = sum w_s O_s / sum w_s l_s
// (attention_combine's maths in base 2; empty slices carry m = -inf and weigh nothing). One wave per
// (head, token, 128/CMB_DSPLIT dims): lane l takes slices l, l + 64, ..., issuing all of a slice's loads
// at once and folding its slices with a running max, so up to 64 slices cost one memory round trip;
// shuffles agree on the max and the sum, and LDS sums the lanes' O. Many small workgroups keep the merge
// short: it runs between two launches, on the critical path of every decode step.
#ifndef CMB_DSPLIT
#define CMB_DSPLIT 8 // workgroups per (head, token), each over 128 / CMB_DSPLIT dims
#endif
#define CMB_DIMS (128 / CMB_DSPLIT) // dims per workgroup (grid z = hd / CMB_DIMS)
extern "C" __global__ void __launch_bounds__(64) gi_decode_combine(GiDecodeArgs a) {
    __shared__ float acc_o[64][CMB_DIMS + 1];
    const int h = blockIdx.x, t = blockIdx.y, d0 = blockIdx.z * CMB_DIMS, lane = threadIdx.x;
    const int hd = a.hd, part = hd + 4;
    const float* p = a.part + ((long long)t * a.n_heads + h) * a.nsplit * part;
    float m = GI_NEG_INF, L = 0.f, o[CMB_DIMS];
#pragma unroll
    for (int i = 0; i < CMB_DIMS; i++) o[i] = 0.f;
    for (int s = lane; s < a.nsplit; s += 64) {
        const float* ps = p + s * part;
        float4 v[CMB_DIMS / 4];
#pragma unroll
        for (int i = 0; i < CMB_DIMS / 4; i++) v[i] = *reinterpret_cast<const float4*>(ps + d0 + 4 * i);
        const float2 ml = *reinterpret_cast<const float2*>(ps + hd);
        if (ml.x == GI_NEG_INF) continue; // an empty slice
        const float mn = fmaxf(m, ml.x);
        const float a_old = __builtin_amdgcn_exp2f(m - mn), a_new = __builtin_amdgcn_exp2f(ml.x - mn);
        m = mn;
        L = L * a_old + ml.y * a_new;
#pragma unroll
        for (int i = 0; i < CMB_DIMS / 4; i++) {
            o[4 * i] = o[4 * i] * a_old + v[i].x * a_new;
            o[4 * i + 1] = o[4 * i + 1] * a_old + v[i].y * a_new;
            o[4 * i + 2] = o[4 * i + 2] * a_old + v[i].z * a_new;
            o[4 * i + 3] = o[4 * i + 3] * a_old + v[i].w * a_new;
        }
    }
    float M = m;
    for (int x = 32; x > 0; x >>= 1) M = fmaxf(M, __shfl_xor(M, x, 64));
    const float w = m == GI_NEG_INF ? 0.f : __builtin_amdgcn_exp2f(m - M);
    float LL = L * w;
    for (int x = 32; x > 0; x >>= 1) LL += __shfl_xor(LL, x, 64);
#pragma unroll
    for (int i = 0; i < CMB_DIMS; i++) acc_o[lane][i] = o[i] * w;
    __syncthreads();
    if (lane < CMB_DIMS) {
        float O = 0.f;
#pragma unroll 8
        for (int k = 0; k < 64; k++) O += acc_o[k][lane];
        a.out[(long long)t * a.out_stride + (long long)h * hd + d0 + lane] = O / LL;
    }
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
    long long kv_head_stride;
    int pos0;              // position of query 0 (keys before it are all visible: chunked prefill)
    int n;                 // query tokens
    int n_heads;
    int n_kv;
    float qscale;          // scale * log2(e), applied to the f32 scores
    int q_f16;
    int out_f16;
    int hd;                // head size (the f32 kernels of gi_attn_f32.hip read it; the MFMA kernels are built per size)
    // int8 cache only (gi_prefill_fwd_i8): kc / vc hold int8 rows in the same element layout; the f32 scale
    // of position t, kv head h is at ks / vs [t*sc_stride + h*sc_head_stride]
    const float* ks;
    const float* vs;
    long long sc_stride;
    long long sc_head_stride;
};

#ifndef PF_WAVES
#define PF_WAVES 8         // waves per workgroup, 32 query rows each
#endif
#define PF_BQ (32 * PF_WAVES) // query rows per workgroup
#define PF_SW (PF_WAVES / 2)  // waves staging each of K and V
// s_waitcnt immediate waiting until at most n vector memory operations are outstanding (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt left at their maxima)
#define GI_VMCNT(n) (0x0F70 | ((n) & 15) | (((n) >> 4) << 14))
// s_waitcnt immediate waiting for this wave's LDS operations (lgkmcnt 0, vmcnt and expcnt at their maxima)
#define GI_LGKMCNT0 0xC07F
#define PF_LPW (16 / PF_SW)   // 1 KB loads per staging wave and tile
#define PF_NBUF 4          // LDS tile buffers
#define PF_BK 64           // keys per tile
#define PF_TILE 16384      // bytes of one K or V tile: 64 rows of 256 bytes
#define PF_RESCALE_LOG2 8.0f
#ifndef PF_KPF
#define PF_KPF 8           // K fragments in flight in the QK loop
#endif
#define GI_LDS __attribute__((address_space(3)))
// Tile staging from HBM straight into LDS (buffer_load_dwordx4 ... lds: lane i's 16 bytes land at
// M0 + 16i). Issued from inline asm, so the compiler does not track these loads: were it to see them, it
// places s_waitcnt vmcnt(0) before every transposing LDS read (ds_read_b64_tr_b16) that it cannot prove
// disjoint from them, which makes each wave wait for the tile it has just requested. The kernels order the
// loads themselves (s_waitcnt vmcnt on the issuing wave, then s_barrier). Vector memory loads retire in
// order, so the compiler's own vmcnt(N) waits for the loads it knows stay correct with these in flight
// (more younger loads only make such a wait stricter).
#ifndef GI_DMA_ASM
#define GI_DMA_ASM 1
#endif
__device__ __forceinline__ u4 gi_rsrc_words(const void* p, long long bytes) {
    const uint32_t n = (uint32_t)(bytes < 0 ? 0 : (bytes > 0x7ffffff0ll ? 0x7ffffff0ll : bytes));
    const unsigned long long b = (unsigned long long)p;
    return u4{(uint32_t)b, (uint32_t)(b >> 32) & 0xffffu, n, (uint32_t)GI_RSRC_FLAGS};
}
__device__ __forceinline__ void gi_stage16(const void* base, long long bytes, GI_LDS void* dst, int voff) {
#if GI_DMA_ASM
    const u4 rs = gi_rsrc_words(base, bytes);
    const uint32_t m0 = (uint32_t)(uintptr_t)dst;
    // (s_nop 0: the one wait state an M0 write needs before an LDS-DMA load reads it; the compiler cannot see
    // the load inside the asm, so it would not insert it)
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(m0) : "memory");
#else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(gi_rsrc(base, bytes), dst, 16, voff, 0, 0, 0);
#endif
}
// int8 cache: the value scale goes into the f16 probabilities times this power of two (undone at the
// end) so that small products stay normal f16; with P <= 2^8 a dequantised |V| up to 127 * 65504 / (2^8 *
// PF_I8_VBIAS) ~ 4000 fits (the reference biases by 2^10 with P <= 1, src/cuda.rs:2416-2420)
#define PF_I8_VBIAS 8.f
typedef short gi_s4 __attribute__((__vector_size__(8))); // 4 f16 as ds_read_b64_tr_b16 returns them

// One workgroup = (head, 256 query rows); wave w of 8 owns rows 32w..32w+31 of the tile. Per 64-key tile:
//   S^T[key, q] = K[key, :] . Q[q, :]       v_mfma_f32_32x32x16_f16, K from LDS (A), Q in registers (B)
//   O^T[d, q]  += V^T[d, key] . P^T[key, q]  V^T from LDS (A, by transposing reads), P^T from S^T (B)
// Software pipeline inside each wave: the softmax of tile t (VALU) runs between the MFMAs of QK for
// tile t+1 and of PV for tile t, which do not depend on it, so the VALU work hides under the matrix core's
// 32-cycle MFMAs instead of following them (a SIMD does not overlap one wave's VALU with another wave's
// back-to-back MFMAs, so the overlap has to come from within the wave).
// Staging: K and V tiles go global -> LDS with direct-to-LDS buffer loads (no registers, no VALU): each of
// the 8 waves moves 4 KB per tile as 4 loads of 1 KB (64 lanes x 16 bytes, written at base + 16*lane).
// Rows are stored unpadded with an XOR swizzle of their 16-byte units (K: unit ^ row%16, V: unit ^
// 4*(row%4)) so the MFMA operand reads hit distinct banks. Iteration t reads V of tile t and K of tile
// t+1; once every wave has passed its barrier tile t-1 is free and tile t+3 streams into its buffer.
// Keys past the cache's end read as zeros (buffer bounds) and are masked.
// K operand: A-row r of S^T block bb holds tile key 32bb + 16(i/2) + 8h + 4(i%2) + j for r = 8i + 4h + j,
// so the 16 values a lane holds per block are exactly the keys its PV B operand needs (k-step 2bb + i/2,
// element 4(i%2) + j). V^T operand: ds_read_b64_tr_b16 gives output lane i of a 16-lane group element
// i%4 of the 8 bytes source lane 4e + i/4 addresses, as its element e; with source lane (e, c) pointing at
// key e, dims 16*(group%2) + 4c of the dim block, lane i receives V[key e][dim i]: the A operand rows.
// Softmax: scores stay raw, scale*log2(e) is folded into the exp2 argument; a row's reference max only
// moves when a tile's max exceeds it by more than 2^8 in probability (then O and l are rescaled), so
// P <= 256 fits f16 and most tiles skip the rescale. Row sums add the f16-rounded P that PV uses
// (v_dot2 against ones). Causal: a wave skips tiles past its last row (keeping every barrier); only
// tiles crossing the diagonal are masked. Work order: the grid is remapped so that each of the 8 XCDs
// (blockIdx round-robin) walks a contiguous run of (kv head, query tile, head) items, longest query
// tiles first, so one kv head's K/V stays in one XCD's L2.
// I8 = true: an int8 cache (the reference's KV8 prefill, src/cuda.rs:2466-2498, 2548-2605): each thread
// loads 16 bytes of a K row and of a V row of the tile into registers one iteration ahead, widens them to
// exact f16 and writes them into the same swizzled LDS layout (so the MFMA operand reads are unchanged),
// and the tile's 64 key and value scales go to LDS beside it. Scores are the integer-key dot products
// times the key scale (QK chains start from zero; s = acc * kscale - m); P V takes f16(p * vscale *
// PF_I8_VBIAS) and the row sum the f16-rounded p, as the reference's pv / pf.
// HD = 64 (attn_prefill_tc<64>, src/cuda.rs:2620): the same kernel with half the QK k-steps and O^T blocks. The
// LDS image keeps the head-128 layout: each 128-byte row sits in a 256-byte slot, its 8 units at the swizzled
// positions the operand reads compute (the staging loads of the other 8 positions are switched off by lane).
template <bool I8, int HD = 128, bool STG = false>
__device__ __forceinline__ void gi_prefill_t(const GiPrefillArgs& a) {
    static_assert(HD == 64 || HD == 128, "head sizes 64, 128 (256: gi_prefill256r)");
    static_assert(!STG || I8, "pre-widened staging: the int8 cache");
    // STG: the int8 cache already widened to exact f16 integers in a workspace (gi_kv_widen, rows [n_kv][len][hd],
    // scales [n_kv][len], the value scales times PF_I8_VBIAS), staged by LDS-DMA as the f16 cache is; else int8
    // tiles are widened through registers (RSTG)
    constexpr bool RSTG = I8 && !STG;
    constexpr int WAVES = PF_WAVES;
    constexpr int BQ = 32 * WAVES;  // query rows per workgroup
    constexpr int SW = WAVES / 2;   // waves staging each of K and V
    constexpr int LPW = 16 / SW;    // 1 KB loads per staging wave and tile
    constexpr int LPT = LPW + (STG ? 1 : 0); // loads per staging wave and tile (STG: plus a quarter of the scales)
    constexpr int BK = PF_BK;       // keys per tile
    constexpr int NBLK = BK / 32;   // S^T blocks of 32 keys
    constexpr int KS = HD / 16;     // QK k-steps
    constexpr int NDB = HD / 32;    // O^T blocks of 32 dims
    __shared__ __attribute__((aligned(1024))) unsigned char smem[PF_NBUF][2][PF_TILE]; // [buffer][K, V]
    __shared__ __attribute__((aligned(16))) float scl[I8 ? PF_NBUF : 1][2][BK];         // int8: [buffer][K, V] scales

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = a.n_heads / a.n_kv;
    const int qtiles = (a.n + BQ - 1) / BQ;
    const int nwg = gridDim.x;
    int j = blockIdx.x;
    if ((nwg & 7) == 0) j = (j & 7) * (nwg >> 3) + (j >> 3);
    const int kvh = j / (qtiles * G);
    const int rest = j % (qtiles * G);
    const int qt = qtiles - 1 - rest / G; // longest query tiles first
    const int h = kvh * G + rest % G;
    const int q0 = qt * BQ;
    const int kv_len = a.pos0 + a.n;
    const int k_lim = min(kv_len, a.pos0 + q0 + BQ); // keys any row of the tile may see
    const int ntiles = (k_lim + BK - 1) / BK;
    const long long kvs = a.kv_stride;

    // ---- staging: the first half of the waves moves K rows, the second half V rows (SW waves each,
    // LPW loads of 1 KB per wave and tile); wave w's load i covers tile rows 4*(LPW*(w%SW) + i)
    // + lane/16, LDS unit lane%16 holding global unit (lane%16) ^ swizzle(row)
    const bool stage_v = wave >= SW;
    const uint16_t* sbase = (stage_v ? a.vc : a.kc) + kvh * a.kv_head_stride;
    int soff[LPW];
    bool sval[LPW]; // head size 64: the lane's LDS unit holds one of the row's 8 units
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        const int r = 4 * (LPW * (wave % SW) + i) + (lane >> 4);
        const int u = (lane & 15) ^ (stage_v ? ((r & 3) << 2) : (r & 15));
        soff[i] = (r * (int)kvs + 8 * u) * 2;
        sval[i] = u < HD / 8;
    }
    auto stage = [&](int t) {
        const int t0 = t * BK;
        const uint16_t* src = sbase + (long long)t0 * kvs;
        const long long bytes = (long long)(kv_len - t0) * kvs * 2;
        unsigned char* dst = &smem[t & (PF_NBUF - 1)][stage_v ? 1 : 0][1024 * LPW * (wave % SW)];
#pragma unroll
        for (int i = 0; i < LPW; i++)
            if (HD == 128 || sval[i]) gi_stage16(src, bytes, (GI_LDS void*)(dst + 1024 * i), soff[i]);
        if constexpr (STG) {
            // this wave's quarter of the tile's 64 scales (16 floats: lanes 0-3, 16 bytes each)
            const float* sp = (stage_v ? a.vs : a.ks) + kvh * a.sc_head_stride + t0;
            if (lane < 4)
                gi_stage16(sp, (long long)(kv_len - t0) * 4, (GI_LDS void*)&scl[t & (PF_NBUF - 1)][stage_v ? 1 : 0][16 * (wave % SW)],
                           64 * (wave % SW) + 16 * lane);
        }
    };
    // int8 staging: thread -> tile row sr, 16-byte chunk sch (dims 16sch..16sch+15) of K and of V; threads
    // 0-63 also take the K scale of key tid, 64-127 the V scale of key tid-64 (times PF_I8_VBIAS)
    // (head size 64: rows of 4 chunks, threads 0-255)
    constexpr int NCH = HD / 16;
    const int sr = tid / NCH, sch = tid % NCH;
    const bool stager = tid < PF_BK * NCH;
    const int8_t* kb8 = reinterpret_cast<const int8_t*>(a.kc) + kvh * a.kv_head_stride;
    const int8_t* vb8 = reinterpret_cast<const int8_t*>(a.vc) + kvh * a.kv_head_stride;
    const float* scb = I8 ? (tid < 64 ? a.ks : a.vs) + kvh * a.sc_head_stride : nullptr;
    u4 rk = u4{0u, 0u, 0u, 0u}, rv = rk;
    float rsc = 0.f;
    // Lanes with sch >= 4 hold their chunk's two 8-byte halves swapped (and write them in that order below):
    // then the 8 lanes of a row that one 16-byte LDS store serves write 8 different units mod 8, all 32
    // banks, where 2sch alone would cover half of them twice.
    const int flip = (sch >> 2) & 1;
    auto load8 = [&](int t) {
        const int t0 = t * PF_BK;
        const int off = sr * (int)kvs + 16 * sch;
        const __amdgpu_buffer_rsrc_t rsk = gi_rsrc(kb8 + (long long)t0 * kvs, (long long)(kv_len - t0) * kvs);
        const __amdgpu_buffer_rsrc_t rsv = gi_rsrc(vb8 + (long long)t0 * kvs, (long long)(kv_len - t0) * kvs);
        if (stager) {
            const u2 k0 = gi_load8(rsk, off + 8 * flip), k1 = gi_load8(rsk, off + 8 - 8 * flip);
            const u2 v0 = gi_load8(rsv, off + 8 * flip), v1 = gi_load8(rsv, off + 8 - 8 * flip);
            rk = u4{k0.x, k0.y, k1.x, k1.y};
            rv = u4{v0.x, v0.y, v1.x, v1.y};
        }
        if (tid < 2 * PF_BK)
            rsc = gi_load4f(gi_rsrc(scb + (long long)t0 * a.sc_stride, (long long)(kv_len - t0) * a.sc_stride * 4),
                            (tid & (PF_BK - 1)) * (int)a.sc_stride * 4);
    };
    auto write8 = [&](int t) {
        unsigned char* K = &smem[t & (PF_NBUF - 1)][0][sr * 256];
        unsigned char* V = &smem[t & (PF_NBUF - 1)][1][sr * 256];
#pragma unroll
        for (int hw = 0; hw < 2; hw++) { // f16 unit 2sch + (hw ^ flip): dims 16sch + 8(hw ^ flip) .. +7
            if (!stager) break;
            const int u = 2 * sch + (hw ^ flip);
            u4 kw, vw;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t xk = gi_i8_in(rk[2 * hw + e]), xv = gi_i8_in(rv[2 * hw + e]);
                kw[2 * e] = i8_f16x2(xk, GI_I8_LO);
                kw[2 * e + 1] = i8_f16x2(xk, GI_I8_HI);
                vw[2 * e] = i8_f16x2(xv, GI_I8_LO);
                vw[2 * e + 1] = i8_f16x2(xv, GI_I8_HI);
            }
            *reinterpret_cast<u4*>(K + ((u ^ (sr & 15)) << 4)) = kw;
            *reinterpret_cast<u4*>(V + ((u ^ ((sr & 3) << 2)) << 4)) = vw;
        }
        if (tid < 2 * PF_BK) scl[t & (PF_NBUF - 1)][tid >> 6][tid & (PF_BK - 1)] = tid < PF_BK ? rsc : rsc * PF_I8_VBIAS;
    };

    // ---- Q as B operands: lane (col = l%32, half = l/32), k-step ks: dims 16ks + 8*half .. +7
    const int qcol = lane & 31, half = lane >> 5;
    const int qrow = q0 + 32 * wave + qcol;      // this lane's query row
    const int qpos = a.pos0 + qrow;              // its position
    // Q is held pre-multiplied by scale*log2(e), so scores come out of the MFMA in log2 units (the f16
    // rounding of the scaled value is the same size as the rounding of Q itself)
    const float qs = a.qscale;
    h8 qf[KS];
    {
        const int qr = qrow < a.n ? qrow : a.n - 1; // rows past n compute garbage that is never written
        if (a.q_f16) {
            const _Float16* qp = (const _Float16*)a.q + (long long)qr * a.q_stride + h * HD + 8 * half;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const h8 x = __builtin_bit_cast(h8, *reinterpret_cast<const u4*>(qp + 16 * ks));
#pragma unroll
                for (int e = 0; e < 8; e++) qf[ks][e] = (_Float16)((float)x[e] * qs);
            }
        } else {
            const float* qp = (const float*)a.q + (long long)qr * a.q_stride + h * HD + 8 * half;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                float4 x0 = *reinterpret_cast<const float4*>(qp + 16 * ks);
                float4 x1 = *reinterpret_cast<const float4*>(qp + 16 * ks + 4);
                qf[ks] = h8{(_Float16)(x0.x * qs), (_Float16)(x0.y * qs), (_Float16)(x0.z * qs), (_Float16)(x0.w * qs),
                            (_Float16)(x1.x * qs), (_Float16)(x1.y * qs), (_Float16)(x1.z * qs), (_Float16)(x1.w * qs)};
            }
        }
    }

    // ---- operand read offsets (bytes within a buffer's K or V tile)
    const int r = lane & 31;
    const int kperm = 16 * ((r >> 3) >> 1) + 8 * ((r >> 2) & 1) + 4 * ((r >> 3) & 1) + (r & 3);
    // K row kperm (block 1 is 32 rows = 8192 bytes further), unit (2ks + half) ^ (kperm % 16)
    //   = 2(ks ^ ky) + (half ^ kperm % 2)
    const int kbase = kperm * 256 + ((half ^ (kperm & 1)) << 4);
    const int ky = (kperm >> 1) & 7;
    const int tg = lane >> 4, ts = lane & 15, te = ts >> 2, tc = ts & 3;
    // V row 8*half + te (+16ks, +4 for the second read), unit 4*(db ^ te) + 2*(tg%2) + tc/2
    const int vbase = (8 * half + te) * 256 + ((2 * (tg & 1) + (tc >> 1)) << 4) + 8 * (tc & 1);

    // ---- per-lane state: O^T (4 dim blocks of 32), reference max (log2 units; tile 0 sets it), row sum
    f16x o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[db][e] = 0.f;
    float m_run = 0.f, l_run = 0.f;
    f16x negm; // -m_run in every element: the C operand that starts each QK chain
#pragma unroll
    for (int e = 0; e < 16; e++) negm[e] = 0.f;

    // S^T of tile t (its K in buffer t%4) minus the row's reference max: each chain starts from C = negm,
    // so the MFMA output is the exp2 argument itself
    // MFMA st of a tile's 16 alternates the two key blocks (k-step st/2, key block st%2)
    auto kfrag = [&](const unsigned char* K, int st) {
        const int reg = st & 1, ksr = st >> 1;
        return *reinterpret_cast<const h8*>(K + 8192 * reg + kbase + 32 * (ksr ^ ky));
    };
    auto qk = [&](int t, f16x* s) {
        const unsigned char* K = &smem[t & (PF_NBUF - 1)][0][0];
        // K fragments stream through a ring of PF_KPF registers, each read PF_KPF MFMAs before its use
        h8 kf[PF_KPF];
#pragma unroll
        for (int st = 0; st < PF_KPF; st++) kf[st] = kfrag(K, st);
        __builtin_amdgcn_sched_barrier(0); // the first PF_KPF reads go out before any of the MFMAs
#pragma unroll
        for (int st = 0; st < 2 * KS; st++) {
            const int ks = st >> 1, bb = st & 1;
            const h8 cur = kf[st % PF_KPF];
            if (st + PF_KPF < 2 * KS) kf[st % PF_KPF] = kfrag(K, st + PF_KPF);
            s[bb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur, qf[ks], ks == 0 ? (I8 ? f16x{} : negm) : s[bb], 0, 0, 0);
        }
    };
    // int8: scores of tile t (its QK sums in s) times their key scales, minus the reference max. Lane holds
    // block bb, element 4i + jj: tile key 32bb + 16(i/2) + 8*half + 4(i%2) + jj
    auto kscale = [&](int t, f16x* s) {
        if constexpr (I8) {
            const float* ksl = &scl[t & (PF_NBUF - 1)][0][8 * half];
#pragma unroll
            for (int bb = 0; bb < 2; bb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 k4 = *reinterpret_cast<const float4*>(ksl + 32 * bb + 16 * (i >> 1) + 4 * (i & 1));
                    s[bb][4 * i] = fmaf(s[bb][4 * i], k4.x, -m_run);
                    s[bb][4 * i + 1] = fmaf(s[bb][4 * i + 1], k4.y, -m_run);
                    s[bb][4 * i + 2] = fmaf(s[bb][4 * i + 2], k4.z, -m_run);
                    s[bb][4 * i + 3] = fmaf(s[bb][4 * i + 3], k4.w, -m_run);
                }
        }
    };

    const int wave_first = a.pos0 + q0 + 32 * wave;  // position of the wave's first row
    const int wave_last = wave_first + 31;
    const int my_tiles = min(ntiles, wave_last / BK + 1); // tiles this wave computes
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));

    // Prologue: tiles 0-2 start loading; tile 0 is waited for and published, and its QK issued. (int8:
    // tiles 0 and 1 are loaded and written, tile 2's loads stay in flight into registers.)
    if constexpr (RSTG) {
        load8(0);
        write8(0);
        if (ntiles > 1) {
            load8(1);
            write8(1);
        }
        if (ntiles > 2) load8(2);
        __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0): this thread's LDS writes are done
    } else {
        stage(0);
        if (ntiles > 1) stage(1);
        if (ntiles > 2) stage(2);
        if (ntiles > 2) __builtin_amdgcn_s_waitcnt(GI_VMCNT(2 * LPT)); // tile 0 is in
        else if (ntiles > 1) __builtin_amdgcn_s_waitcnt(GI_VMCNT(LPT));
        else __builtin_amdgcn_s_waitcnt(GI_VMCNT(0));
    }
    asm volatile("s_barrier" ::: "memory");
    // One pipeline step: tile it's softmax and PV, with QK of tile it+1 into sn (past this wave's last
    // tile that QK reads a stale buffer and is never used). No branch separates the QK MFMAs from the
    // VALU work they hide.
    // row max of a tile's scores (relative to m_run) over the row's two lane halves (lanes l and l + 32,
    // exchanged by a VALU lane swap, no LDS round trip)
    auto rowmax = [&](const f16x* sc) {
        float mx = GI_NEG_INF;
#pragma unroll
        for (int bb = 0; bb < NBLK; bb++)
#pragma unroll
            for (int e = 0; e < 16; e++) mx = fmaxf(mx, sc[bb][e]);
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_int(mx), __float_as_int(mx), false, false);
        return fmaxf(__int_as_float(p[0]), __int_as_float(p[1]));
    };
    // One pipeline step for tile it (scores s, their row max mx): the rare rescale first, then one
    // branch-free block that issues QK of tile it+1 into sn, computes tile it's probabilities k-step by
    // k-step under those MFMAs and the PV MFMAs of tile it, and ends with tile it+1's row max (mx on exit),
    // so that the next step can start its exp2 work at once. Past this wave's last tile the QK reads a
    // stale buffer and is never used.
    auto step = [&](int it, f16x* s, f16x* sn, float& mx) {
        const bool up = mx > PF_RESCALE_LOG2 || it == 0;
        if (__builtin_amdgcn_ballot_w64(up)) {
            // some row's max moved (tile 0: every row takes its first max): shift the reference by delta,
            // rescale O and l (alpha = 1 for the other rows; O and l are still 0 at tile 0) and this tile's
            // scores; the next tile's QK starts from the new reference
            const float delta = up ? mx : 0.f;
            const float alpha = __builtin_amdgcn_exp2f(-fmaxf(delta, 0.f));
            m_run += delta;
#pragma unroll
            for (int e = 0; e < 16; e++) negm[e] = -m_run;
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; db++) gi_acc_scale<false>(o[db], alpha);
#pragma unroll
            for (int bb = 0; bb < NBLK; bb++) s[bb] -= delta;
        }
        qk(it + 1, sn);
        // probabilities of k-step ks feed the PV MFMAs of k-step ks
        const unsigned char* V = &smem[it & (PF_NBUF - 1)][1][0];
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            const int bb = ks >> 1;
            h8 pf;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const int i = 2 * (ks & 1) + (e >> 2), jj = e & 3;
                const float p0 = __builtin_amdgcn_exp2f(s[bb][4 * i + jj]);
                const float p1 = __builtin_amdgcn_exp2f(s[bb][4 * i + jj + 1]);
                const _Float16 h0 = (_Float16)p0, h1 = (_Float16)p1;
                if constexpr (I8) { // P V takes p times the value scale; the row sum the rounded p
                    const float* vsl = &scl[it & (PF_NBUF - 1)][1][32 * bb + 16 * (i >> 1) + 8 * half + 4 * (i & 1) + jj];
                    pf[e] = (_Float16)(p0 * vsl[0]);
                    pf[e + 1] = (_Float16)(p1 * vsl[1]);
                } else {
                    pf[e] = h0;
                    pf[e + 1] = h1;
                }
                l_run = __builtin_amdgcn_fdot2(h2{h0, h1}, h2{(_Float16)1.f, (_Float16)1.f}, l_run, false);
            }
#pragma unroll
            for (int db = 0; db < NDB; db++) {
                const unsigned char* vp = V + vbase + ((db ^ te) << 6) + 4096 * ks;
                gi_s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((GI_LDS gi_s4*)(vp));
                gi_s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((GI_LDS gi_s4*)(vp + 1024));
                h8 vf = __builtin_shufflevector(__builtin_bit_cast(h4x, lo), __builtin_bit_cast(h4x, hi),
                                                0, 1, 2, 3, 4, 5, 6, 7);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf, o[db], 0, 0, 0);
            }
        }
        kscale(it + 1, sn);
        mx = rowmax(sn); // unmasked: a diagonal tile recomputes it after masking
        // Instruction order of the QK phase: every QK MFMA is followed by the read of the K fragment PF_KPF
        // MFMAs on (the compiler otherwise reads each fragment just before its MFMA). Interleaving the
        // softmax VALU or the V reads by further groups measured no better.
#pragma unroll
        for (int i = 0; i < 2 * KS; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                          // MFMA
            if (i + PF_KPF < 2 * KS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // its K refill
        }
    };
    // Iteration it: before the barrier each wave waits for its own loads of tile it+1 (tile it+2's may
    // stay in flight); the barrier publishes the tile and tells that every wave is done with tile it-1,
    // whose buffer then takes tile it+3. Barriers are bare s_barrier (__syncthreads' release fence would
    // also wait for tile it+2's loads); the memory clobber keeps LDS accesses on their side.
    float mx = GI_NEG_INF;
    // int8: the registers loaded in iteration it-1 (tile it+2) are written into its buffer (free: every wave
    // has passed tile it-2) right after the barrier, and tile it+3's loads go out; a wave's LDS writes are
    // complete before the next barrier publishes them.
    auto iteration = [&](int it, f16x* s, f16x* sn) {
        if constexpr (RSTG) {
            __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0)
        } else {
            if (it + 2 < ntiles) __builtin_amdgcn_s_waitcnt(GI_VMCNT(LPT)); // tile it+2's loads may stay in flight
            else __builtin_amdgcn_s_waitcnt(GI_VMCNT(0));
        }
        asm volatile("s_barrier" ::: "memory");
        if constexpr (RSTG) {
            if (it + 2 < ntiles) {
                write8(it + 2);
                if (it + 3 < ntiles) load8(it + 3);
            }
        } else {
            if (it + 3 < ntiles) stage(it + 3);
        }
        if (it < my_tiles) {
            const int t0 = it * BK;
            if (t0 + BK - 1 > wave_first) { // the tile crosses the diagonal (or the end) somewhere in the wave
                // lane holds, for query qcol: block bb, element 4i + jj -> tile key 32bb + 16(i/2) + 8*half + 4(i%2) + jj
                const int lim = qpos - t0 - 8 * half;
#pragma unroll
                for (int bb = 0; bb < NBLK; bb++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int jj = 0; jj < 4; jj++)
                            if (32 * bb + 16 * (i >> 1) + 4 * (i & 1) + jj > lim) s[bb][4 * i + jj] = GI_NEG_INF;
                mx = rowmax(s);
            }
            step(it, s, sn, mx);
        }
    };
    f16x sa[NBLK], sb[NBLK]; // scores of alternate tiles
    if (my_tiles > 0) {
        qk(0, sa);
        kscale(0, sa);
        mx = rowmax(sa);
    }
    for (int it = 0; it < ntiles; it += 2) {
        iteration(it, sa, sb);
        if (it + 1 < ntiles) iteration(it + 1, sb, sa);
    }

    // ---- normalise and write: lane holds query qcol, dims 32db + 8i + 4*half + jj
    float l = l_run + __shfl_xor(l_run, 32, 64);
    if (qrow < a.n) {
        const float inv = (I8 ? 1.f / PF_I8_VBIAS : 1.f) / l;
        if (a.out_f16) {
            _Float16* op = (_Float16*)a.out + (long long)qrow * a.out_stride + h * HD + 4 * half;
#pragma unroll
            for (int db = 0; db < NDB; db++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    h4x v = h4x{(_Float16)(o[db][4 * i] * inv), (_Float16)(o[db][4 * i + 1] * inv),
                                (_Float16)(o[db][4 * i + 2] * inv), (_Float16)(o[db][4 * i + 3] * inv)};
                    *reinterpret_cast<h4x*>(op + 32 * db + 8 * i) = v;
                }
        } else {
            float* op = (float*)a.out + (long long)qrow * a.out_stride + h * HD + 4 * half;
#pragma unroll
            for (int db = 0; db < NDB; db++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    *reinterpret_cast<float4*>(op + 32 * db + 8 * i) =
                        make_float4(o[db][4 * i] * inv, o[db][4 * i + 1] * inv, o[db][4 * i + 2] * inv, o[db][4 * i + 3] * inv);
        }
    }
}

// ---------------------------------------------------------------- prefill, head size 256, 16 rows per wave
// One workgroup per (head, 128 query rows): 8 waves of 16 rows, each with all 256 output dims, so QK and the
// softmax are computed once per row (the reference's attention_prefill_tc256 splits the output dims over
// two blocks that both compute QK, src/cuda.rs:2622-2623). On v_mfma_f32_16x16x32_f16, per 64-key tile:
//  - S^T (4 blocks of 16 keys x 16 queries) = K Q^T over 8 k-steps of 32 dims, each chain starting from
//    C = -(reference max). Lane l holds query column c = l%16 and rows 4g + r (g = l/16) of each block.
//    A-row rho of key block kb reads tile key 8(rho/4) + 4(kb%2) + 32(kb/2) + rho%4, so the lane's rows
//    are keys 32(kb/2) + 8g + 4(kb%2) + r: exactly the keys 32kp + 8g + e (kp = kb/2, e = 4(kb%2) + r) it
//    holds in the P^T operand of k-step kp of P V, with no data movement.
//  - O^T (16 blocks of 16 dims x 16 queries) += V^T P^T: per 16-dim block one MFMA for each 32 keys, V^T
//    from two transposing reads (keys 8g..8g+3 and 8g+4..8g+7 of the 32, 16 dims).
// LDS image of a K or V tile (32 KB): row r holds key r%64, dims 128(r/64) .. +127 (256 bytes), its 16-byte
// units XOR-swizzled (pf256r_swz_k / pf256r_swz_v). Per tile a wave issues 64 MFMAs against 64 KB of LDS
// operand reads, twice the bytes per flop of the head-size-128 kernel's 32-row waves.
__device__ __forceinline__ int pf256r_swz_k(int r) { return (r & 15) ^ (((r >> 4) & 1) << 2); }
__device__ __forceinline__ int pf256r_swz_v(int r) { return ((r & 3) << 2) | (((r >> 3) & 1) << 1); }
#define PF256R_WAVES 8
#define PF256R_ROWS 16
#define PF256R_BQ (PF256R_ROWS * PF256R_WAVES) // query rows per workgroup
// K and V rings: NKBUF and NVBUF buffers of one tile each (NKBUF + NVBUF <= 5 in 160 KB of LDS). Iteration
// it reads K of tile it+1 (its QK) and V of tile it (its P V); after its barrier the buffers of K(it) and
// V(it-1) have no reader left, so it refills them with K(it + NKBUF) and V(it + NVBUF - 1): each tile is
// issued NKBUF - 1 (K) or NVBUF - 1 (V) iterations before its use. Half the waves stage K, half V, and
// each waits for its own loads only, then the barrier publishes them.
// FMT 1 (the int8 cache, attention_prefill_tc256 with KV8, src/cuda.rs:2466-2498, 2548-2605) and 2 (the 4-bit
// cache, with KV4, src/cuda.rs:2495-2514): the staging waves load the compressed rows into registers, widen them
// to f16 (int8: the exact integers; 4-bit: f16((n - 8) * scale)) and write the same swizzled f16 image, one tile
// ahead of the barrier that publishes it. int8 also stages each tile's key and value scales: a score is the dot
// product with the integer key times the key's scale, P V takes f16(p * vscale * 2^10), the row sum the f16 p,
// and the output is divided by 2^10.
template <int NKBUF, int NVBUF, int FMT = 0, bool STG = false>
__device__ __forceinline__ void gi_prefill256r(const GiPrefillArgs& a) {
    static_assert(NKBUF >= 2 && NVBUF >= 2 && NKBUF + NVBUF <= 5, "K and V rings within 160 KB");
    static_assert(!STG || FMT == 1, "pre-widened staging: the int8 cache (the 4-bit one widens to the f16 kernel's input)");
    // STG: the int8 cache already widened to exact f16 integers in a workspace (gi_kv_widen: rows [n_kv][len][256],
    // raw scales [n_kv][len]), staged by LDS-DMA as the f16 cache is
    constexpr bool REG = FMT != 0 && !STG; // staging through registers
    constexpr int HD = 256, WAVES = PF256R_WAVES, BQ = PF256R_BQ, BK = 64;
    constexpr int SW = WAVES / 2;            // waves staging each of K and V
    constexpr int LPW = (BK / 2) / SW;       // 1 KB loads per staging wave and tile (K or V: BK * 512 bytes)
    constexpr int LPT = LPW + (STG ? 1 : 0); // loads per staging wave and tile (STG: plus a quarter of the scales)
    constexpr int KS = HD / 32;              // QK k-steps
    constexpr int NKB = BK / 16;             // S^T blocks of 16 keys
    constexpr int NDB = HD / 16;             // O^T blocks of 16 dims
    constexpr int TILE = BK * 512;           // bytes of one K or V tile image
    constexpr int VPF = REG ? 4 : 0;         // V^T fragments read ahead in P V (0: the compiler's order)
    __shared__ __attribute__((aligned(1024))) unsigned char smem[(NKBUF + NVBUF) * TILE];
    __shared__ __attribute__((aligned(16))) float sc_sh[FMT == 1 ? NKBUF + NVBUF : 1][BK]; // int8: tile scales
    auto kbuf = [&](int t) { return smem + (t % NKBUF) * TILE; };
    auto vbuf = [&](int t) { return smem + (NKBUF + t % NVBUF) * TILE; };
    auto kscl = [&](int t) { return &sc_sh[t % NKBUF][0]; };
    auto vscl = [&](int t) { return &sc_sh[FMT == 1 ? NKBUF + t % NVBUF : 0][0]; };
    // wait until at most n (0..2) of this wave's tile loads are outstanding
    auto wait_tiles = [&](int n) {
        if constexpr (REG) return; // (register staging: the compiler waits for the loads it issued)
        if (n >= 2) __builtin_amdgcn_s_waitcnt(GI_VMCNT(2 * LPT));
        else if (n == 1) __builtin_amdgcn_s_waitcnt(GI_VMCNT(LPT));
        else __builtin_amdgcn_s_waitcnt(GI_VMCNT(0));
    };
    static_assert(NKBUF <= 4 && NVBUF <= 4, "wait_tiles covers two tiles in flight past the one waited for");

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = a.n_heads / a.n_kv;
    const int qtiles = (a.n + BQ - 1) / BQ;
    const int nwg = gridDim.x;
    int j = blockIdx.x;
    if ((nwg & 7) == 0) j = (j & 7) * (nwg >> 3) + (j >> 3); // each XCD a contiguous run of items
    const int kvh = j / (qtiles * G);
    const int rest = j % (qtiles * G);
    const int qt = qtiles - 1 - rest / G; // longest query tiles first
    const int h = kvh * G + rest % G;
    const int q0 = qt * BQ;
    const int kv_len = a.pos0 + a.n;
    const int k_lim = min(kv_len, a.pos0 + q0 + BQ);
    const int ntiles = (k_lim + BK - 1) / BK;
    const long long kvs = a.kv_stride;

    // ---- staging: wave w's load i covers image rows 4*(LPW*(w%SW) + i) + lane/16 (row r = key r%BK, dims
    // 128*(r/BK)..), LDS unit lane%16 holding global unit (lane%16) ^ swizzle(r). K: the key's low 4 bits with bit 4 folded into bit 2, so
    // that the 16 rows one K fragment read touches (keys 8(c/4) + c%4 (+4), c = 0..15: low 4 bits repeat at
    // c and c + 8) fall on 16 different unit positions. V: (key % 4) << 2 with bit 3 into bit 1, so that lane
    // groups g and g + 1 of a transposing read (keys 8g + te and 8g + 8 + te) use disjoint banks.
    const bool stage_v = wave >= SW;
    const uint16_t* sbase = (stage_v ? a.vc : a.kc) + kvh * a.kv_head_stride;
    int soff[LPW];
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        const int r = 4 * (LPW * (wave % SW) + i) + (lane >> 4);
        const int u = (lane & 15) ^ (stage_v ? pf256r_swz_v(r) : pf256r_swz_k(r));
        soff[i] = ((r & (BK - 1)) * (int)kvs + 128 * (r / BK) + 8 * u) * 2;
    }
    // this wave's share of tile t (its K if it stages K, else its V)
    auto stage = [&](int t) {
        const int t0 = t * BK;
        const uint16_t* src = sbase + (long long)t0 * kvs;
        const long long bytes = (long long)(kv_len - t0) * kvs * 2;
        unsigned char* dst = (stage_v ? vbuf(t) : kbuf(t)) + 1024 * LPW * (wave % SW);
#pragma unroll
        for (int i = 0; i < LPW; i++) gi_stage16(src, bytes, (GI_LDS void*)(dst + 1024 * i), soff[i]);
        if constexpr (STG) {
            // this wave's quarter of the tile's 64 scales (16 floats: lanes 0-3, 16 bytes each)
            static_assert(SW * 16 == BK, "a quarter of the scales per staging wave");
            const float* sp = (stage_v ? a.vs : a.ks) + kvh * a.sc_head_stride + t0;
            if (lane < 4)
                gi_stage16(sp, (long long)(kv_len - t0) * 4, (GI_LDS void*)((stage_v ? vscl(t) : kscl(t)) + 16 * (wave % SW)),
                           64 * (wave % SW) + 16 * lane);
        }
    };
    // ---- register staging (FMT 1, 2): staging lane l takes a quarter (l/16) of key 16(wave % SW) + l%16's row,
    // values 64 quarter .. +63, i.e. image row key + 64(quarter/2), units 8(quarter%2) .. +7 (swizzled as above):
    // the 16 lanes of a quarter write 16 keys' rows, whose swizzles put their 16-byte units on distinct banks
    // (one quarter per lane and key instead measured 12% slower). These LDS writes, not the widening, are what
    // the register path costs against the f16 cache's LDS-DMA staging (widening without the writes: 0.77 ms at
    // 8192 tokens, 16/2; the writes without the widening: 1.31 ms).
    // int8 rows: 4 16-byte loads and the key's f32 scale (quarter 0's lane); 4-bit rows: 2 16-byte loads and the
    // two f16 scales of its groups. `pend` holds one tile's loads from its issue to its widening.
    const int skey = 16 * (wave % SW) + (lane & 15), squart = lane >> 4;
    const int srow = skey + BK * (squart >> 1);
    struct Pend { u4 w[FMT == 1 ? 4 : 2]; uint32_t sc; int t; } pend;
    pend.t = -1;
    const unsigned char* sbase8 = reinterpret_cast<const unsigned char*>(stage_v ? a.vc : a.kc) + kvh * a.kv_head_stride;
    const void* scbase = nullptr;
    if constexpr (FMT == 1) scbase = (stage_v ? a.vs : a.ks) + kvh * a.sc_head_stride;
    if constexpr (FMT == 2) scbase = reinterpret_cast<const uint16_t*>(stage_v ? a.vs : a.ks) + kvh * a.sc_head_stride;
    auto issue = [&](int t) {
        const int t0 = t * BK;
        const __amdgpu_buffer_rsrc_t r = gi_rsrc(sbase8 + (long long)t0 * kvs, (long long)(kv_len - t0) * kvs);
        if constexpr (FMT == 1) {
#pragma unroll
            for (int i = 0; i < 4; i++) pend.w[i] = gi_load16(r, skey * (int)kvs + 64 * squart + 16 * i);
            const float* sp = reinterpret_cast<const float*>(scbase) + (long long)t0 * a.sc_stride;
            pend.sc = __builtin_amdgcn_raw_buffer_load_b32(gi_rsrc(sp, (long long)(kv_len - t0) * a.sc_stride * 4),
                                                           skey * (int)a.sc_stride * 4, 0, 0);
        } else {
#pragma unroll
            for (int i = 0; i < 2; i++) pend.w[i] = gi_load16(r, skey * (int)kvs + 32 * squart + 16 * i);
            const uint16_t* sp = reinterpret_cast<const uint16_t*>(scbase) + (long long)t0 * a.sc_stride;
            pend.sc = __builtin_amdgcn_raw_buffer_load_b32(gi_rsrc(sp, (long long)(kv_len - t0) * a.sc_stride * 2),
                                                           (skey * (int)a.sc_stride + 2 * squart) * 2, 0, 0);
        }
        pend.t = t;
    };
    // widen the pending tile into its buffer (the next barrier publishes it, after this wave's LDS writes are
    // waited for)
    auto commit = [&]() {
        if (pend.t < 0) return;
        const int t = pend.t;
        unsigned char* img = stage_v ? vbuf(t) : kbuf(t);
        const int swz = stage_v ? pf256r_swz_v(srow) : pf256r_swz_k(srow);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            u4 h;
            if constexpr (FMT == 1) {
                const uint32_t x0 = gi_i8_in(pend.w[i >> 1][2 * (i & 1)]), x1 = gi_i8_in(pend.w[i >> 1][2 * (i & 1) + 1]);
                h = u4{i8_f16x2(x0, GI_I8_LO), i8_f16x2(x0, GI_I8_HI), i8_f16x2(x1, GI_I8_LO), i8_f16x2(x1, GI_I8_HI)};
            } else {
                const uint32_t x = pend.w[i >> 2][i & 3];
                const h2x sc = __builtin_bit_cast(h2x, (i >> 2) ? (pend.sc >> 16) * 0x10001u : (pend.sc & 0xffffu) * 0x10001u);
                h = u4{q4_f16x2(x >> 4, x, 0, sc), q4_f16x2(x >> 4, x, 1, sc), q4_f16x2(x >> 4, x, 2, sc),
                       q4_f16x2(x >> 4, x, 3, sc)};
            }
            const int unit = (8 * (squart & 1) + i) ^ swz;
            *reinterpret_cast<GI_LDS u4*>((GI_LDS unsigned char*)img + srow * 256 + (unit << 4)) = h;
        }
        if constexpr (FMT == 1)
            if (squart == 0) (stage_v ? vscl(t) : kscl(t))[skey] = __uint_as_float(pend.sc);
        pend.t = -1;
    };
    // iteration it's staging: the pending tile (K: it + NKBUF into K(it)'s buffer; V: it + NVBUF - 1 into
    // V(it-1)'s; both free since the barrier of it) is widened, and the loads of the next one are issued, so
    // each tile's loads have a whole iteration to land and its widening runs among the wave's MFMAs
    auto restage = [&](int it) {
        commit();
        if (!stage_v && it + NKBUF + 1 < ntiles) issue(it + NKBUF + 1);
        if (stage_v && it + NVBUF < ntiles) issue(it + NVBUF);
    };

    // ---- Q as B operands: lane (column c, k-group g), k-step ks: dims 32ks + 8g .. +7, times scale*log2(e)
    const int c = lane & 15, g = lane >> 4;
    const int qrow = q0 + PF256R_ROWS * wave + c;
    const int qpos = a.pos0 + qrow;
    const float qs = a.qscale;
    h8 qf[KS];
    {
        const int qr = qrow < a.n ? qrow : a.n - 1; // rows past n compute garbage that is never written
        if (a.q_f16) {
            const _Float16* qp = (const _Float16*)a.q + (long long)qr * a.q_stride + h * HD + 8 * g;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const h8 x = __builtin_bit_cast(h8, *reinterpret_cast<const u4*>(qp + 32 * ks));
#pragma unroll
                for (int e = 0; e < 8; e++) qf[ks][e] = (_Float16)((float)x[e] * qs);
            }
        } else {
            const float* qp = (const float*)a.q + (long long)qr * a.q_stride + h * HD + 8 * g;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const float4 x0 = *reinterpret_cast<const float4*>(qp + 32 * ks);
                const float4 x1 = *reinterpret_cast<const float4*>(qp + 32 * ks + 4);
                qf[ks] = h8{(_Float16)(x0.x * qs), (_Float16)(x0.y * qs), (_Float16)(x0.z * qs), (_Float16)(x0.w * qs),
                            (_Float16)(x1.x * qs), (_Float16)(x1.y * qs), (_Float16)(x1.z * qs), (_Float16)(x1.w * qs)};
            }
        }
    }

    // ---- operand read offsets (bytes within a buffer's K or V image)
    // K: block kb, k-step ks: key krow + 4(kb%2) + 32(kb/2) (krow = 8(c/4) + c%4), image half ks/4, unit
    // 4(ks%4) + g swizzled
    const int krow = 8 * (c >> 2) + (c & 3);
    auto kfrag = [&](const unsigned char* K, int st) { // MFMA st of a tile's NKB*KS: block st%NKB, k-step st/NKB
        const int kb = st % NKB, ks = st / NKB;
        const int key = krow + 4 * (kb & 1) + 32 * (kb >> 1);
        const int unit = (4 * (ks & 3) + g) ^ pf256r_swz_k(key);
        return *reinterpret_cast<const h8*>(K + (key + BK * (ks >> 2)) * 256 + (unit << 4));
    };
    // V: block db (dims 16db..), keys 8g + te (+4): image row 32*(db/8) + 8g + te, unit 2*(db%8) + tc/2 swizzled,
    // plus 8 bytes for odd tc (te = (lane%16)/4, tc = lane%4); the +4 rows of the second read keep the swizzle
    // (BK = 64: k-step kp of P V takes keys 32kp + ..)
    const int te = c >> 2, tc = c & 3;
    const int vbase = (8 * g + te) * 256 + 8 * (tc & 1);
    auto vfrag = [&](const unsigned char* V, int db, int kp) {
        const int off = vbase + 8192 * kp + BK * 256 * (db >> 3) +
                        (((2 * (db & 7) + (tc >> 1)) ^ pf256r_swz_v(8 * g + te)) << 4);
        gi_s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((GI_LDS gi_s4*)(V + off));
        gi_s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((GI_LDS gi_s4*)(V + off + 1024));
        return __builtin_shufflevector(__builtin_bit_cast(h4x, lo), __builtin_bit_cast(h4x, hi), 0, 1, 2, 3, 4, 5,
                                       6, 7);
    };

    // ---- per-lane state: O^T (16 blocks of 16 dims; this lane dims 16db + 4g + r), reference max, row sum
    f4 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; db++) o[db] = f4{0.f, 0.f, 0.f, 0.f};
    float m_run = 0.f, l_run = 0.f;
    f4 negm = f4{0.f, 0.f, 0.f, 0.f}; // -m_run: the C operand that starts each QK chain

    // this lane's keys of a tile: 32(kb/2) + 8g + 4(kb%2) + r, 4 consecutive per block
    auto key_scales = [&](const float* sc, f4* out) {
#pragma unroll
        for (int kb = 0; kb < NKB; kb++)
            out[kb] = *reinterpret_cast<const f4*>(sc + 32 * (kb >> 1) + 8 * g + 4 * (kb & 1));
    };
    auto qk = [&](int t, f4* s) {
        const unsigned char* K = kbuf(t);
        h8 kf[PF_KPF];
#pragma unroll
        for (int st = 0; st < PF_KPF; st++) kf[st] = kfrag(K, st);
        __builtin_amdgcn_sched_barrier(0);
        const f4 zero = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < NKB * KS; st++) {
            const int kb = st % NKB, ks = st / NKB;
            const h8 cur = kf[st % PF_KPF];
            if (st + PF_KPF < NKB * KS) kf[st % PF_KPF] = kfrag(K, st + PF_KPF);
            s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur, qf[ks], ks == 0 ? (FMT == 1 ? zero : negm) : s[kb], 0, 0,
                                                           0);
        }
        if constexpr (FMT == 1) { // the score: the integer key's dot product times its scale, less the max
            f4 ksv[NKB];
            key_scales(kscl(t), ksv);
#pragma unroll
            for (int kb = 0; kb < NKB; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) s[kb][r] = fmaf(s[kb][r], ksv[kb][r], -m_run);
        }
    };
    auto rowmax = [&](const f4* sc) {
        float mx = GI_NEG_INF;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) mx = fmaxf(mx, fmaxf(fmaxf(sc[kb][0], sc[kb][1]), fmaxf(sc[kb][2], sc[kb][3])));
        return rows_max(mx);
    };
    const int wave_first = a.pos0 + q0 + PF256R_ROWS * wave; // position of the wave's first row
    const int wave_last = wave_first + PF256R_ROWS - 1;
    const int my_tiles = min(ntiles, wave_last / BK + 1);
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));

    // one step: the rare rescale, then QK of tile it+1 into sn under tile it's probabilities and P V, and tile
    // it+1's row max (mx on exit)
    auto step = [&](int it, f4* s, f4* sn, float& mx) {
        const bool up = mx > PF_RESCALE_LOG2 || it == 0;
        if (__builtin_amdgcn_ballot_w64(up)) {
            const float delta = up ? mx : 0.f;
            const float alpha = __builtin_amdgcn_exp2f(-fmaxf(delta, 0.f));
            m_run += delta;
            negm = f4{-m_run, -m_run, -m_run, -m_run};
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; db++) gi_acc_scale<false>(o[db], alpha);
#pragma unroll
            for (int kb = 0; kb < NKB; kb++) s[kb] -= delta;
        }
        qk(it + 1, sn);
        h8 pf[NKB / 2]; // k-step kp: keys 32kp + 8g + e, e = 4(kb%2) + r for block kb = 2kp + kb%2
        f4 vsv[FMT == 1 ? NKB : 1];
        if constexpr (FMT == 1) key_scales(vscl(it), vsv);
#pragma unroll
        for (int kb = 0; kb < NKB; kb++)
#pragma unroll
            for (int r = 0; r < 4; r += 2) {
                const float p0 = __builtin_amdgcn_exp2f(s[kb][r]), p1 = __builtin_amdgcn_exp2f(s[kb][r + 1]);
                const _Float16 h0 = (_Float16)p0, h1 = (_Float16)p1;
                if constexpr (FMT == 1) { // P V weights: f16(p * vscale * 2^10)
                    pf[kb >> 1][4 * (kb & 1) + r] = (_Float16)(p0 * (vsv[kb][r] * 1024.f));
                    pf[kb >> 1][4 * (kb & 1) + r + 1] = (_Float16)(p1 * (vsv[kb][r + 1] * 1024.f));
                } else {
                    pf[kb >> 1][4 * (kb & 1) + r] = h0;
                    pf[kb >> 1][4 * (kb & 1) + r + 1] = h1;
                }
                l_run = __builtin_amdgcn_fdot2(h2{h0, h1}, h2{(_Float16)1.f, (_Float16)1.f}, l_run, false);
            }
        const unsigned char* V = vbuf(it);
        if constexpr (VPF > 0) {
            // register staging: V^T fragments stream through a ring of VPF registers, each read VPF MFMAs
            // before its use (the f16 kernel measured faster with the compiler's own order)
            constexpr int NPV = (NKB / 2) * NDB;
            h8 vq[VPF > 0 ? VPF : 1];
#pragma unroll
            for (int i = 0; i < VPF; i++) vq[i] = vfrag(V, i % NDB, i / NDB);
#pragma unroll
            for (int i = 0; i < NPV; i++) {
                const int kp = i / NDB, db = i % NDB;
                const h8 cur = vq[i % VPF];
                if (i + VPF < NPV) vq[i % VPF] = vfrag(V, (i + VPF) % NDB, (i + VPF) / NDB);
                o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur, pf[kp], o[db], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int kp = 0; kp < NKB / 2; kp++)
#pragma unroll
                for (int db = 0; db < NDB; db++)
                    o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vfrag(V, db, kp), pf[kp], o[db], 0, 0, 0);
        }
        mx = rowmax(sn);
#pragma unroll
        for (int i = 0; i < NKB * KS; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i + PF_KPF < NKB * KS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if constexpr (VPF > 0) { // then the first V reads, and each P V MFMA followed by its ring refill
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * VPF, 0);
#pragma unroll
            for (int i = 0; i < (NKB / 2) * NDB; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (i + VPF < (NKB / 2) * NDB) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            }
        }
    };

    // prologue: K of tiles 0..NKBUF-1 and V of tiles 0..NVBUF-2 start loading; K(0) is waited for and
    // published (the rest are waited for by the iterations that first read them)
    const int last_k0 = min(NKBUF - 1, ntiles - 1), last_v0 = min(NVBUF - 2, ntiles - 1);
    for (int t = 0; t <= (stage_v ? last_v0 : last_k0); t++) {
        if constexpr (REG) {
            issue(t);
            commit();
        } else {
            stage(t);
        }
    }
    if constexpr (REG) { // the tile iteration 0 widens
        if (!stage_v && NKBUF < ntiles) issue(NKBUF);
        if (stage_v && NVBUF - 1 < ntiles) issue(NVBUF - 1);
        __builtin_amdgcn_s_waitcnt(GI_LGKMCNT0);
    }
    if (!stage_v) wait_tiles(last_k0);
    asm volatile("s_barrier" ::: "memory");
    float mx = GI_NEG_INF;
    auto iteration = [&](int it, f4* s, f4* sn) {
        // K waves need K(it+1), having issued up to K(it + NKBUF - 1); V waves need V(it), issued up to
        // V(it + NVBUF - 2)
        if (stage_v) wait_tiles(max(min(it + NVBUF - 2, ntiles - 1) - it, 0));
        else wait_tiles(max(min(it + NKBUF - 1, ntiles - 1) - (it + 1), 0));
        if constexpr (REG) __builtin_amdgcn_s_waitcnt(GI_LGKMCNT0); // the widened tile's writes, before they publish
        asm volatile("s_barrier" ::: "memory");
        if constexpr (!REG) {
            if (!stage_v && it + NKBUF < ntiles) stage(it + NKBUF);    // into K(it)'s buffer
            if (stage_v && it + NVBUF - 1 < ntiles) stage(it + NVBUF - 1); // into V(it-1)'s buffer
        }
        if (it < my_tiles) {
            const int t0 = it * BK;
            if (t0 + BK - 1 > wave_first) { // the tile crosses the diagonal somewhere in the wave
                const int lim = qpos - t0;
#pragma unroll
                for (int kb = 0; kb < NKB; kb++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (32 * (kb >> 1) + 8 * g + 4 * (kb & 1) + r > lim) s[kb][r] = GI_NEG_INF;
                mx = rowmax(s);
            }
            step(it, s, sn, mx);
        }
        if constexpr (REG) restage(it);
    };
    f4 sa[NKB], sb[NKB];
    if (my_tiles > 0) {
        qk(0, sa);
        mx = rowmax(sa);
    }
    for (int it = 0; it < ntiles; it += 2) {
        iteration(it, sa, sb);
        if (it + 1 < ntiles) iteration(it + 1, sb, sa);
    }

    // ---- normalise and write: lane holds query c, dims 16db + 4g + r
    const float l = rows_sum(l_run);
    if (qrow < a.n) {
        const float inv = FMT == 1 ? (1.f / 1024.f) / l : 1.f / l;
        if (a.out_f16) {
            _Float16* op = (_Float16*)a.out + (long long)qrow * a.out_stride + h * HD + 4 * g;
#pragma unroll
            for (int db = 0; db < NDB; db++)
                *reinterpret_cast<h4x*>(op + 16 * db) = h4x{(_Float16)(o[db][0] * inv), (_Float16)(o[db][1] * inv),
                                                            (_Float16)(o[db][2] * inv), (_Float16)(o[db][3] * inv)};
        } else {
            float* op = (float*)a.out + (long long)qrow * a.out_stride + h * HD + 4 * g;
#pragma unroll
            for (int db = 0; db < NDB; db++)
                *reinterpret_cast<float4*>(op + 16 * db) =
                    make_float4(o[db][0] * inv, o[db][1] * inv, o[db][2] * inv, o[db][3] * inv);
        }
    }
}

extern "C" __global__ void __launch_bounds__(64 * PF_WAVES, 1) gi_prefill_fwd(GiPrefillArgs a) { gi_prefill_t<false>(a); }
extern "C" __global__ void __launch_bounds__(64 * PF_WAVES, 1) gi_prefill_fwd_i8(GiPrefillArgs a) { gi_prefill_t<true>(a); }
extern "C" __global__ void __launch_bounds__(64 * PF_WAVES, 1) gi_prefill_fwd_h64(GiPrefillArgs a) { gi_prefill_t<false, 64>(a); }
extern "C" __global__ void __launch_bounds__(64 * PF_WAVES, 1) gi_prefill_fwd_h64_i8(GiPrefillArgs a) { gi_prefill_t<true, 64>(a); }
// the int8 cache pre-widened by gi_kv_widen, staged as the f16 cache is
extern "C" __global__ void __launch_bounds__(64 * PF_WAVES, 1) gi_prefill_fwd_i8s(GiPrefillArgs a) { gi_prefill_t<true, 128, true>(a); }
extern "C" __global__ void __launch_bounds__(64 * PF_WAVES, 1) gi_prefill_fwd_h64_i8s(GiPrefillArgs a) { gi_prefill_t<true, 64, true>(a); }
#ifndef PF256R_KBUF
#define PF256R_KBUF 2 // K tile buffers of gi_prefill_fwd_h256r
#endif
#ifndef PF256R_VBUF
#define PF256R_VBUF 2 // V tile buffers of gi_prefill_fwd_h256r
#endif
extern "C" __global__ void __launch_bounds__(64 * PF256R_WAVES, 1) gi_prefill_fwd_h256r(GiPrefillArgs a) {
    gi_prefill256r<PF256R_KBUF, PF256R_VBUF>(a);
}
extern "C" __global__ void __launch_bounds__(64 * PF256R_WAVES, 1) gi_prefill_fwd_h256r_i8(GiPrefillArgs a) {
    gi_prefill256r<PF256R_KBUF, PF256R_VBUF, 1>(a);
}
extern "C" __global__ void __launch_bounds__(64 * PF256R_WAVES, 1) gi_prefill_fwd_h256r_q4(GiPrefillArgs a) {
    gi_prefill256r<PF256R_KBUF, PF256R_VBUF, 2>(a);
}
// the int8 cache pre-widened by gi_kv_widen (the 4-bit cache pre-widened runs gi_prefill_fwd_h256r itself)
extern "C" __global__ void __launch_bounds__(64 * PF256R_WAVES, 1) gi_prefill_fwd_h256r_i8s(GiPrefillArgs a) {
    gi_prefill256r<PF256R_KBUF, PF256R_VBUF, 1, true>(a);
}

// ------------------------------------------------------------------------------------------------ KV store

// Arguments of gi_qk_norm_rope (must match gi_attn_host.cpp).
struct GiRopeArgs {
    float* qkv;            // packed rows [q (n_heads*hd) | k (n_kv*hd) | v (n_kv*hd)] f32, row_stride apart
    const float* qn;       // RMSNorm weights of q heads [hd] (null: no norm)
    const float* kn;       // of k heads
    uint16_t* kc;          // f16 caches: position t, kv head h at t*kv_stride + h*kv_head_stride
    uint16_t* vc;
    const float* ff;       // RoPE frequency factors [rope_dim/2] (null: none)
    const int* posp;       // device position (overrides pos0 when non-null)
    long long row_stride;
    long long kv_stride;
    long long kv_head_stride;
    int pos0;
    int n;                 // tokens
    int n_heads;
    int n_kv;
    int hd;                // 64, 128, 256, or a multiple of 16 up to 112 (the lane-masked form)
    int rope_dim;          // rotated dims (even, <= hd); the rest pass unchanged
    float base;
    float eps;
    int neox;              // pairs (i, i + rope_dim/2); otherwise (2i, 2i+1)
    int fmt;               // cache format: 0 f16; 1 int8 (kc / vc as bytes, same element offsets) with f32 scales
                           // (position t, kv head h at t*sc_stride + h*sc_head_stride); 2 the 4-bit cache (head
                           // size 256: kv strides in bytes, a row of 128 bytes; ks / vs hold 8 f16 scales a row,
                           // sc strides in f16 elements)
    float* ks;
    float* vs;
    long long sc_stride;
    long long sc_head_stride;
    int ctx_cap;           // positions the cache holds: rows at positions outside [0, ctx_cap) are not stored
    int pad_;
};

// Reference semantics: qk_norm_rope (src/cuda.rs:437-486) with an f16 cache (kv_store, src/cuda.rs:312-362).
// A q or k head: RMSNorm (ss = sum of squares over the head, scale = rsqrt(ss/hd + eps), times the
// weights), then RoPE on rope_dim/2 pairs (freq_i = base^(-2i/rope_dim) / ff[i], angle = pos * freq_i, all
// f32), written back into qkv; a k head also goes to the K cache. A v head goes to the V cache unchanged.
// Cache values are rounded to nearest even. One workgroup per (token, group of ROPE_HEADS heads of the
// packed row: q heads, then k, then v): the pairs' sines and cosines depend only on the position, so the
// workgroup computes them once into LDS for all its heads; each wave loads its ROPE_HEADS/4 heads at once
// and takes them one at a time through a per-wave LDS row (any two dims can pair).
#define ROPE_HEADS 16
// The normalized 256-point Walsh-Hadamard transform of a row held 4 values per lane (lane l: values 4l..4l+3):
// kv4_fwht's stages (src/cuda.rs:242-256) in its order, h = 1, 2 inside the lane, h = 4..128 across lanes
// l and l ^ (h/4). Each stage gives the lower element a + c and the upper one a - c, single f32 operations as
// the reference's, so the result is bit-identical to it; then every value times 1/16.
__device__ __forceinline__ void gi_fwht256(float __attribute__((ext_vector_type(4))) & x, int lane) {
    float t;
    t = x[0]; x[0] = t + x[1]; x[1] = t - x[1];
    t = x[2]; x[2] = t + x[3]; x[3] = t - x[3];
    t = x[0]; x[0] = t + x[2]; x[2] = t - x[2];
    t = x[1]; x[1] = t + x[3]; x[3] = t - x[3];
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const bool upper = lane & m;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float p = __shfl_xor(x[j], m, 64);
            x[j] = upper ? p - x[j] : x[j] + p;
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) x[j] *= 0.0625f;
}

// One head row (PER values per lane) into a cache row. f16: rounded to nearest even. int8 (kv_store's KV8,
// src/cuda.rs:333-339): dd = max|x| / 127, each value rint(x * (1/dd)) (0 when dd is 0), dd to the scale.
// 4-bit (kv_store's KV4, src/cuda.rs:340-357; PER = 4, the row already rotated): per group of 32 values (8
// lanes) dh = f16(max|x| / 7), inv = 1/dh (0 when dh is 0), q = clamp(rint(x * inv), -7, 7) + 8; lane l writes
// the 2 bytes of values 4l..4l+3 (value 2i in byte i's low nibble), the group's first lane its f16 scale.
template <int PER>
__device__ __forceinline__ void gi_store_row(const GiRopeArgs& a, uint16_t* cache, float* scale, int pos, int kh,
                                             const float __attribute__((ext_vector_type(PER))) x, int lane) {
    if (pos < 0 || pos >= a.ctx_cap) return; // (a device position past the capacity writes nothing)
    const long long off = (long long)pos * a.kv_stride + (long long)kh * a.kv_head_stride;
    const bool act = PER * lane < a.hd; // (lanes past a lane-masked head's dims hold zeros and store nothing)
    if (a.fmt == 0) {
        typedef _Float16 hv __attribute__((ext_vector_type(PER)));
        if (act) *reinterpret_cast<hv*>(cache + off + PER * lane) = __builtin_convertvector(x, hv);
        return;
    }
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < PER; j++) amax = fmaxf(amax, fabsf(x[j]));
    if constexpr (PER == 4) {
        if (a.fmt == 2) {
            for (int m = 4; m > 0; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
            const _Float16 dh = (_Float16)__fdiv_rn(amax, 7.f);
            const float dd = (float)dh, inv = dd != 0.f ? __fdiv_rn(1.f, dd) : 0.f;
            uint32_t w = 0;
#pragma unroll
            for (int j = 0; j < 4; j++)
                w |= (uint32_t)(fminf(fmaxf(rintf(x[j] * inv), -7.f), 7.f) + 8.f) << (4 * j);
            *reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(cache) + off + 2 * lane) = (uint16_t)w;
            if ((lane & 7) == 0)
                reinterpret_cast<_Float16*>(scale)[(long long)pos * a.sc_stride + (long long)kh * a.sc_head_stride +
                                                   (lane >> 3)] = dh;
            return;
        }
    }
    for (int m = 32; m > 0; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
    const float dd = __fdiv_rn(amax, 127.f), inv = dd != 0.f ? __fdiv_rn(1.f, dd) : 0.f;
    typedef int8_t bv __attribute__((ext_vector_type(PER)));
    bv q;
#pragma unroll
    for (int j = 0; j < PER; j++) q[j] = (int8_t)__float2int_rn(x[j] * inv);
    if (act) *reinterpret_cast<bv*>(reinterpret_cast<int8_t*>(cache) + off + PER * lane) = q;
    if (lane == 0) scale[(long long)pos * a.sc_stride + (long long)kh * a.sc_head_stride] = dd;
}

// PER = hd / 64 values per lane, dims PER*lane .. PER*lane + PER - 1 (one 4, 8 or 16-byte access per row).
// MASKED (PER = 2): any even head size up to 128 (the f32 kernels' head sizes): lanes past hd / 2 hold zeros and
// neither load nor store.
template <int PER, bool MASKED = false>
__device__ __forceinline__ void gi_qk_norm_rope_t(const GiRopeArgs& a, float (*cs_sh)[2], float (*row_sh)[256]) {
    typedef float fv __attribute__((ext_vector_type(PER)));
    static_assert(!MASKED || PER == 2, "the lane-masked form: two values per lane");
    const int HD = MASKED ? a.hd : 64 * PER;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool act = !MASKED || PER * lane < HD; // the lane holds dims of the head
    const int items = a.n_heads + 2 * a.n_kv;
    const int b = blockIdx.y, h0 = blockIdx.x * ROPE_HEADS;
    const int pos = (a.posp ? *a.posp : a.pos0) + b;
    const int half = a.rope_dim >> 1;
    if (tid < half && h0 < a.n_heads + a.n_kv) { // (a workgroup of v heads only rotates nothing)
        float freq = powf(a.base, -2.0f * (float)tid / (float)a.rope_dim);
        if (a.ff) freq /= a.ff[tid];
        float s, c;
        sincosf((float)pos * freq, &s, &c);
        cs_sh[tid][0] = c;
        cs_sh[tid][1] = s;
    }
    __syncthreads();
    float* row = a.qkv + (long long)b * a.row_stride;
    float* sh = row_sh[wave];
    // all of this wave's head rows are loaded up front (more bytes in flight per wave), then processed
    constexpr int HPW = ROPE_HEADS / 4;
    fv v[HPW];
#pragma unroll
    for (int k = 0; k < HPW; k++) {
        const int h = h0 + wave + 4 * k;
        v[k] = fv{};
        if (h < items && act) v[k] = *reinterpret_cast<const fv*>(row + (long long)h * HD + PER * lane); // q, k, v heads in turn
    }
#pragma unroll
    for (int k = 0; k < HPW; k++) {
        const int h = h0 + wave + 4 * k;
        if (h >= items) break;
        if (h >= a.n_heads + a.n_kv) { // a v head: into the cache (the 4-bit cache: rotated first)
            fv x = v[k];
            if constexpr (PER == 4)
                if (a.fmt == 2) gi_fwht256(x, lane);
            gi_store_row<PER>(a, a.vc, a.vs, pos, h - a.n_heads - a.n_kv, x, lane);
            continue;
        }
        fv x = v[k];
        if (a.qn) {
            const float* w = h < a.n_heads ? a.qn : a.kn;
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < PER; j++) ss = fmaf(x[j], x[j], ss);
            for (int m = 32; m > 0; m >>= 1) ss += __shfl_xor(ss, m, 64);
            const float scale = __frsqrt_rn(ss / (float)HD + a.eps);
            const fv wv = act ? *reinterpret_cast<const fv*>(w + PER * lane) : fv{};
#pragma unroll
            for (int j = 0; j < PER; j++) x[j] = x[j] * scale * wv[j];
        }
        if (act) *reinterpret_cast<fv*>(sh + PER * lane) = x;
        __builtin_amdgcn_wave_barrier();
        for (int i = lane; i < half; i += 64) {
            const int ia = a.neox ? i : 2 * i, ib = a.neox ? i + half : 2 * i + 1;
            const float p = sh[ia], q = sh[ib], c = cs_sh[i][0], s = cs_sh[i][1];
            sh[ia] = p * c - q * s;
            sh[ib] = p * s + q * c;
        }
        __builtin_amdgcn_wave_barrier();
        if (act) x = *reinterpret_cast<const fv*>(sh + PER * lane);
        // the 4-bit cache (src/cuda.rs:472-479): q and k heads rotated alike, so their dot products are kept
        if constexpr (PER == 4)
            if (a.fmt == 2) gi_fwht256(x, lane);
        if (act) *reinterpret_cast<fv*>(row + (long long)h * HD + PER * lane) = x;
        if (h >= a.n_heads) gi_store_row<PER>(a, a.kc, a.ks, pos, h - a.n_heads, x, lane);
        __builtin_amdgcn_wave_barrier(); // the row buffer is reused by the wave's next head
    }
}
extern "C" __global__ void __launch_bounds__(256) gi_qk_norm_rope(GiRopeArgs a) {
    __shared__ float cs_sh[128][2];  // cos, sin of pair i
    __shared__ float row_sh[4][256]; // a head row per wave
    if (a.hd == 64) gi_qk_norm_rope_t<1>(a, cs_sh, row_sh);
    else if (a.hd == 128) gi_qk_norm_rope_t<2>(a, cs_sh, row_sh);
    else if (a.hd == 256) gi_qk_norm_rope_t<4>(a, cs_sh, row_sh);
    else gi_qk_norm_rope_t<2, true>(a, cs_sh, row_sh);
}

// ------------------------------------------------------------------------------- output rotation (4-bit cache)

// Arguments of gi_hadamard_rows (must match gi_attn_host.cpp).
struct GiHadamardArgs {
    float* x;              // rows of segs * 256 floats, row_stride apart
    long long row_stride;
    int rows;
    int segs;              // 256-value segments a row
};

// hadamard_rows with block 256 and no signs (src/cuda.rs:4675-4693), as the layer applies it to the attention
// output of a 4-bit cache (src/cuda.rs:9765-9768): every 256-value segment of a row, in place, through the
// normalized Walsh-Hadamard transform (the same stages as kv4_fwht; its rsqrtf(256) is 1/16). One wave per
// segment, 4 values a lane.
extern "C" __global__ void __launch_bounds__(256) gi_hadamard_rows(GiHadamardArgs a) {
    const int lane = threadIdx.x & 63;
    const long long seg = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (seg >= (long long)a.rows * a.segs) return;
    float* p = a.x + (seg / a.segs) * a.row_stride + (seg % a.segs) * 256 + 4 * lane;
    float __attribute__((ext_vector_type(4))) v = *reinterpret_cast<float __attribute__((ext_vector_type(4)))*>(p);
    gi_fwht256(v, lane);
    *reinterpret_cast<float __attribute__((ext_vector_type(4)))*>(p) = v;
}

// ------------------------------------------------------------------------------------------- cache growth

// Arguments of gi_kv_relayout (must match gi_attn_host.cpp). Strides in bytes.
struct GiRelayoutArgs {
    const unsigned char* src;
    unsigned char* dst;
    long long src_stride;      // between positions
    long long src_head_stride; // between kv heads
    long long dst_stride;
    long long dst_head_stride;
    long long n_units;         // n_kv * n_rows * units_per_row
    int n_rows;
    int units_per_row;
    int unit;                  // bytes per unit: 16 or 4
    int pad_;
};
// Cache growth (LayerCache::resize, src/cuda.rs:9962-9976, which the reference does as one contiguous copy of
// `keep` rows): rows (position t < n_rows, kv head h) of one layout copied into another, e.g. a head-major
// cache [n_kv][cap][hd] into one of a larger capacity, whose rows all move. Thread -> one 16-byte (or 4-byte)
// unit; consecutive threads walk a head's rows in order, so both sides stream whole rows.
extern "C" __global__ void __launch_bounds__(256) gi_kv_relayout(GiRelayoutArgs a) {
    for (long long i = blockIdx.x * 256ll + threadIdx.x; i < a.n_units; i += (long long)gridDim.x * 256) {
        const int u = (int)(i % a.units_per_row);
        const long long r = i / a.units_per_row;
        const long long t = r % a.n_rows, h = r / a.n_rows;
        const unsigned char* sp = a.src + t * a.src_stride + h * a.src_head_stride + (long long)u * a.unit;
        unsigned char* dp = a.dst + t * a.dst_stride + h * a.dst_head_stride + (long long)u * a.unit;
        if (a.unit == 16) *reinterpret_cast<u4*>(dp) = *reinterpret_cast<const u4*>(sp);
        else *reinterpret_cast<uint32_t*>(dp) = *reinterpret_cast<const uint32_t*>(sp);
    }
}

// ------------------------------------------------------------------------------------- pre-widened prefill staging

// Arguments of gi_kv_widen (must match gi_attn_host.cpp).
struct GiWidenArgs {
    const unsigned char* kc;   // int8 rows (fmt 1) or 4-bit rows of hd / 2 bytes (fmt 2)
    const unsigned char* vc;
    const void* ks;            // fmt 1: f32 scale per (position, kv head); fmt 2: hd / 32 f16 scales a row
    const void* vs;
    uint16_t* kw;              // f16 rows [n_kv][n_rows][hd]
    uint16_t* vw;
    float* ksw;                // fmt 1: f32 scales [n_kv][n_rows] (values times vbias)
    float* vsw;
    long long kv_stride;       // bytes between positions
    long long kv_head_stride;  // bytes between kv heads
    long long sc_stride;       // scale elements between positions
    long long sc_head_stride;  // scale elements between kv heads
    int n_rows;
    int n_kv;
    int hd;
    int fmt;
    float vbias;
    int pad_;
};
// The compressed cache widened once per prefill launch into a workspace that the prefill kernels stage by LDS-DMA,
// as they stage the f16 cache (the widening inside the prefill costs its LDS writes from registers). int8: the
// exact f16 integers and the row scales (the prefill applies them as over the int8 cache); 4-bit: f16((n - 8) *
// scale), the values attention_prefill_tc256 with KV4 feeds its tensor cores (src/cuda.rs:2495-2514). Thread -> one
// 16-byte unit (8 values) of a K and a V row, consecutive threads along a head's rows.
extern "C" __global__ void __launch_bounds__(256) gi_kv_widen(GiWidenArgs a) {
    const int upr = a.hd / 8; // units per row
    const long long n_units = (long long)a.n_kv * a.n_rows * upr;
    for (long long i = blockIdx.x * 256ll + threadIdx.x; i < n_units; i += (long long)gridDim.x * 256) {
        const int u = (int)(i % upr);
        const long long r = i / upr;
        const int t = (int)(r % a.n_rows), h = (int)(r / a.n_rows);
        const long long src = t * a.kv_stride + h * a.kv_head_stride;
        const long long se = t * a.sc_stride + h * a.sc_head_stride;
        u4 kw, vw;
        if (a.fmt == 1) {
            const u2 k8 = *reinterpret_cast<const u2*>(a.kc + src + 8 * u);
            const u2 v8 = *reinterpret_cast<const u2*>(a.vc + src + 8 * u);
            const uint32_t k0 = gi_i8_in(k8.x), k1 = gi_i8_in(k8.y), v0 = gi_i8_in(v8.x), v1 = gi_i8_in(v8.y);
            kw = u4{i8_f16x2(k0, GI_I8_LO), i8_f16x2(k0, GI_I8_HI), i8_f16x2(k1, GI_I8_LO), i8_f16x2(k1, GI_I8_HI)};
            vw = u4{i8_f16x2(v0, GI_I8_LO), i8_f16x2(v0, GI_I8_HI), i8_f16x2(v1, GI_I8_LO), i8_f16x2(v1, GI_I8_HI)};
            if (u == 0) {
                a.ksw[r] = reinterpret_cast<const float*>(a.ks)[se];
                a.vsw[r] = reinterpret_cast<const float*>(a.vs)[se] * a.vbias;
            }
        } else {
            // values 8u .. 8u + 7: bytes 4u .. 4u + 3 (value 2i in byte i's low nibble), scale group u / 4
            const uint32_t k4 = *reinterpret_cast<const uint32_t*>(a.kc + src + 4 * u);
            const uint32_t v4 = *reinterpret_cast<const uint32_t*>(a.vc + src + 4 * u);
            const uint16_t kb = reinterpret_cast<const uint16_t*>(a.ks)[se + u / 4];
            const uint16_t vb = reinterpret_cast<const uint16_t*>(a.vs)[se + u / 4];
            const h2x ksc = __builtin_bit_cast(h2x, (uint32_t)kb * 0x10001u), vsc = __builtin_bit_cast(h2x, (uint32_t)vb * 0x10001u);
            kw = u4{q4_f16x2(k4 >> 4, k4, 0, ksc), q4_f16x2(k4 >> 4, k4, 1, ksc), q4_f16x2(k4 >> 4, k4, 2, ksc),
                    q4_f16x2(k4 >> 4, k4, 3, ksc)};
            vw = u4{q4_f16x2(v4 >> 4, v4, 0, vsc), q4_f16x2(v4 >> 4, v4, 1, vsc), q4_f16x2(v4 >> 4, v4, 2, vsc),
                    q4_f16x2(v4 >> 4, v4, 3, vsc)};
        }
        *reinterpret_cast<u4*>(a.kw + r * a.hd + 8 * u) = kw;
        *reinterpret_cast<u4*>(a.vw + r * a.hd + 8 * u) = vw;
    }
}

// ------------------------------------------------------------------------------------------------ f32 fallback
#include "gi_attn_f32.hip"
