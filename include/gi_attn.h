/* gi_attn.h — C ABI of the MI355X (gfx950) attention path: split-K flash decoding and causal flash
 * prefill over a grouped-query KV cache (f16, int8 or 4-bit).
 *
 * This is the drop-in boundary for ghost-infer's attention operator. In the reference the engine's
 * layer loop calls GpuModel::attention (src/cuda.rs:8448-8541), which launches NVRTC-compiled kernels
 * through Kernels::launch3 (src/cuda.rs:5746-5762). Here a Rust (or C, C++, Python ctypes) caller binds
 * these functions instead; kernels come from an offline-built gfx950 code object loaded with
 * hipModuleLoad.
 *
 * Conventions shared by every entry point (the reference's, src/cuda.rs:5377-5413, 8403-8541):
 *  - All tensor pointers are device pointers owned by the caller; no entry point allocates device
 *    memory. Work is enqueued on `stream` (a hipStream_t; NULL = the null stream) without host sync.
 *  - Return 0 on success. On failure the return is non-zero (GI_EINVAL for a bad argument, otherwise the
 *    hipError_t value) and gi_last_error() gives "HIP <what> failed: <text> (<code>)" or the argument
 *    problem, as the reference's Api::check builds "CUDA {what} failed: {text} ({r})"
 *    (src/cuda.rs:5058-5068). The message is per thread.
 *  - Layouts: query/output rows hold head h at element h*hd of the row (row strides in elements). The
 *    KV cache is two f16 buffers (IEEE binary16 bits); the row of position t, kv head h starts at element
 *    t*kv_stride + h*kv_head_stride. The reference's layout [position][n_kv][hd] (src/cuda.rs:365-369)
 *    is kv_stride = n_kv*hd, kv_head_stride = hd (pass 0 for hd). The head-major layout
 *    [n_kv][capacity][hd] is kv_stride = hd, kv_head_stride = capacity*hd: each head's rows are
 *    contiguous, which spreads a head's stream evenly over the HBM channels (the decode kernel is
 *    fastest with it). Strides are multiples of 8 elements and pointers 16-byte aligned.
 *  - Causality: token b of a call sits at position pos0 + b and attends to keys 0..pos0+b.
 *  - Device positions (posp, graph replay): no entry point reports a device position that overruns the
 *    cache, since the host never sees it. The decode kernels (which gi_attention* use whenever posp is
 *    set) clamp *posp into [0, ctx_cap - n_tok] and return the attention at the clamped position; the
 *    cache writes store no row at a position outside [0, ctx_cap). A caller that can overrun checks its
 *    position on the host before replaying (the reference trusts *posp the same way, src/cuda.rs:8686-8712).
 *  - hd is 64, 128 or 256 with the f16 and the int8 caches, and 256 with the 4-bit cache (the *_q4 entry
 *    points); also 16, 32, 48, 80, 96 or 112 with the f16 and the int8 caches, on f32 kernels (the reference's
 *    f32 fallback, attention_partial and attention_prefill, src/cuda.rs:1866-2041); n_heads must be a multiple
 *    of n_kv. Head size 64 is attention_partial_gqa at a head size that is a multiple of 32
 *    (src/cuda.rs:8419-8422) and attention_prefill_tc64 (src/cuda.rs:2620, dispatched at
 *    src/cuda.rs:8452-8456); 256 the reference's wide heads (attention_partial_gqa's hd 256 branch
 *    src/cuda.rs:1762-1781, attention_prefill_tc256 src/cuda.rs:2622-2623, attention_decode_tc256
 *    src/cuda.rs:2625-2802).
 */
#ifndef GI_ATTN_H
#define GI_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GI_EINVAL (-1)

/* element types of gi_attn_prefill's query and output */
#define GI_F32 0
#define GI_F16 1

/* Load the code object (path to gi_attn_gfx950.hsaco; NULL = $GI_CODE_OBJECT if set, else the file
 * beside this library) on the current device. Optional: every entry point loads it on first use per device.
 * Replaces: Kernels::binary + compile_on (src/cuda.rs:5485-5655), which NVRTC-compile KERNELS and
 * resolve the functions by name. */
int gi_init(const char* code_object_path);

/* Last error message of the calling thread ("" if none). Replaces Api::check's String
 * (src/cuda.rs:5058-5068). */
const char* gi_last_error(void);

/* Slice plan of a decode call: keys per slice (`chunk`) and slices per token (`nsplit`) for tokens whose
 * largest span is max_span. Counterpart of att_want / att_chunk / max_splits (src/cuda.rs:8426-8444),
 * re-chosen for 256 CUs: about one workgroup per CU in total, slices as short as that allows in whole wave tiles
 * (32 keys; 16 at hd 256; the int8 kernels' 64) and at least one tile per wave (128 keys; 64 at hd 256; int8 256).
 * The plan of the f16 cache (the int8 and 4-bit kernels may take other slices). */
int gi_attn_decode_plan(int max_span, int n_tok, int n_heads, int n_kv, int hd, int* chunk, int* nsplit);

/* Bytes of workspace gi_attn_decode needs for n_tok tokens whose spans reach at most ctx_cap keys (the
 * slice partials, [token][head][slice][hd + 4] f32: O, max, sum, 2 pad; 16-byte aligned). Covers the int8
 * entry points too. The counterpart of the session's att_part buffer (GpuSession, src/cuda.rs:9826-9870).
 * The workspace needs no initialisation; calls that share one must be ordered (one stream). */
size_t gi_attn_decode_workspace_bytes(int ctx_cap, int n_tok, int n_heads, int n_kv, int hd);

/* Decode / verify attention for n_tok tokens (one generated token, or a speculative verify block that
 * is causal within itself). q: f32 rows (q_stride elements apart); out: f32 rows. When posp is non-NULL
 * the position is read from device memory (*posp replaces pos0; graph replay) and the grid is sized for
 * ctx_cap keys, so one launch shape serves every position up to ctx_cap - n_tok; otherwise ctx_cap is
 * ignored. The kernel clamps *posp into [0, ctx_cap - n_tok], so a stale or wrong device position reads no
 * key past ctx_cap (it gives the attention at the clamped position instead of an error). Replaces:
 * attention_partial_gqa + attention_combine, launched by GpuModel::attention's split path (src/cuda.rs:1684-1865,
 * src/cuda.rs:2806-2836, src/cuda.rs:8478-8538). */
int gi_attn_decode(void* stream, const float* q, long long q_stride, const uint16_t* kc, const uint16_t* vc,
                   long long kv_stride, long long kv_head_stride, float* out, long long out_stride, void* workspace,
                   size_t workspace_bytes, int pos0, const int* posp, int ctx_cap, int n_tok, int n_heads, int n_kv,
                   int hd, float scale);

/* gi_attn_decode without a workspace: the slice partials go to a fixed 16 MiB array in device memory that the
 * library's code object holds on each device (from its load until the process ends), so the call allocates
 * nothing and takes no scratch argument. No counterpart in the reference; it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Shapes whose
 * partials exceed 16 MiB (n_tok * n_heads * slices * (hd + 4) * 4 bytes; config 2 needs 1.1 MB, an 8-token
 * verify at 32768 keys 8.7 MB; with the default plan of about 256 workgroups no shape needs more than ~9 MB)
 * are rejected with GI_EINVAL. Every call on one device shares that array:
 * calls that may overlap on one device (several streams, or several host threads) race and must not be
 * issued. */
int gi_attn_decode_noalloc(void* stream, const float* q, long long q_stride, const uint16_t* kc, const uint16_t* vc,
                           long long kv_stride, long long kv_head_stride, float* out, long long out_stride, int pos0,
                           const int* posp, int ctx_cap, int n_tok, int n_heads, int n_kv, int hd, float scale);

/* gi_attn_decode over an int8 KV cache: kc / vc hold int8 rows in the element layout above (kv_stride and
 * kv_head_stride multiples of 16), and position t, kv head h has the f32 scales ks / vs [t*sc_stride +
 * h*sc_head_stride] (value = int8 * scale); sc_stride = sc_head_stride = 0 means the reference's [position]
 * [n_kv] (sc_stride = n_kv, sc_head_stride = 1). Scores are (q*scale) . k_int8 * ks, the exp-sum is of the
 * unscaled probabilities and each value row is weighted by probability * vs. Replaces: attention_partial_gqa
 * + attention_combine compiled with KV8 (src/cuda.rs:209-226, src/cuda.rs:1684-1865, src/cuda.rs:2806-2836). */
int gi_attn_decode_i8(void* stream, const float* q, long long q_stride, const int8_t* kc, const int8_t* vc,
                      const float* ks, const float* vs, long long kv_stride, long long kv_head_stride,
                      long long sc_stride, long long sc_head_stride, float* out, long long out_stride, void* workspace,
                      size_t workspace_bytes, int pos0, const int* posp, int ctx_cap, int n_tok, int n_heads, int n_kv,
                      int hd, float scale);

/* gi_attn_decode over the 4-bit KV cache (head size 256; the reference's --kv q4 format, src/cuda.rs:226-256,
 * 340-357): position t, kv head h has a row of 128 bytes at kc / vc + t*kv_stride + h*kv_head_stride (strides in
 * bytes, multiples of 16; kv_head_stride 0 means 128), value 2i in byte i's low nibble and 2i + 1 in its high one,
 * each stored as q + 8, and 8 f16 scales (one per 32 values) at ks / vs + t*sc_stride + h*sc_head_stride (f16
 * elements, even; ks / vs 4-byte aligned; both 0 mean the reference's [position][n_kv][8]). A value is f16((n - 8) * scale). The rows hold
 * rotated vectors (gi_qk_norm_rope_q4 rotates q and k alike and v in the store), so q must be the rotated
 * queries and out holds rotated rows: gi_hadamard_rows turns them back. Replaces: attention_decode_tc256 compiled
 * with KV4 (src/cuda.rs:2625-2802) + attention_combine, as GpuModel::attention dispatches it for 256-wide heads
 * (src/cuda.rs:8478-8538). The workspace is gi_attn_decode_workspace_bytes(..., hd = 256). */
int gi_attn_decode_q4(void* stream, const float* q, long long q_stride, const uint8_t* kc, const uint8_t* vc,
                      const uint16_t* ks, const uint16_t* vs, long long kv_stride, long long kv_head_stride,
                      long long sc_stride, long long sc_head_stride, float* out, long long out_stride, void* workspace,
                      size_t workspace_bytes, int pos0, const int* posp, int ctx_cap, int n_tok, int n_heads, int n_kv,
                      float scale);

/* Causal prefill attention for n tokens at positions pos0..pos0+n-1 whose K/V rows are already in the
 * cache (keys 0..pos0+n-1 are read; pos0 > 0 is a chunk of a longer prompt). q: rows of q_dtype
 * (GI_F32 or GI_F16); out: rows of out_dtype. Replaces: attention_prefill_tc128 (src/cuda.rs:2408-2621), and
 * attention_prefill_tc64 / attention_prefill_tc256 at hd 64 / 256 (src/cuda.rs:2620-2623), launched by
 * GpuModel::attention for batches of >= 16 tokens (src/cuda.rs:8452-8466). */
int gi_attn_prefill(void* stream, const void* q, int q_dtype, long long q_stride, const uint16_t* kc,
                    const uint16_t* vc, long long kv_stride, long long kv_head_stride, void* out, int out_dtype,
                    long long out_stride, int pos0, int n, int n_heads, int n_kv, int hd, float scale);

/* gi_attn_prefill over an int8 KV cache (layouts and scales as gi_attn_decode_i8). The keys enter the
 * scores as exact integers times their scale; P V takes f16(p * vs) and the row sum the f16-rounded p.
 * Dequantised values must stay within |v| < 4000 (the f16 range of p * vs with p <= 256); the output is
 * O / 2^10 / l. hd 64, 128 or 256. Replaces: attention_prefill_tc64/128/256 compiled with KV8
 * (src/cuda.rs:2408-2623, int8 staging src/cuda.rs:2466-2498). */
int gi_attn_prefill_i8(void* stream, const void* q, int q_dtype, long long q_stride, const int8_t* kc, const int8_t* vc,
                       const float* ks, const float* vs, long long kv_stride, long long kv_head_stride,
                       long long sc_stride, long long sc_head_stride, void* out, int out_dtype, long long out_stride,
                       int pos0, int n, int n_heads, int n_kv, int hd, float scale);

/* gi_attn_prefill over the 4-bit cache (head size 256; layouts as gi_attn_decode_q4): the tiles are widened to
 * the f16 values f16((n - 8) * scale) and the rest is the f16 cache's prefill. q: the rotated queries; out: rotated
 * rows (gi_hadamard_rows turns them back). Replaces: attention_prefill_tc256 compiled with KV4 (src/cuda.rs:
 * 2495-2514, 2622-2623). */
int gi_attn_prefill_q4(void* stream, const void* q, int q_dtype, long long q_stride, const uint8_t* kc,
                       const uint8_t* vc, const uint16_t* ks, const uint16_t* vs, long long kv_stride,
                       long long kv_head_stride, long long sc_stride, long long sc_head_stride, void* out, int out_dtype,
                       long long out_stride, int pos0, int n, int n_heads, int n_kv, float scale);

/* Causal prefill in f32 (no f16 rounding of Q or P; f32 MFMA operands and accumulation) over the f16 cache or, with
 * kv_int8, the int8 cache (ks / vs and the scale strides as gi_attn_prefill_i8), head sizes 16 to 128 in steps of 16.
 * Replaces: attention_prefill (src/cuda.rs:1934-2041), which GpuModel::attention launches for prompts when the
 * tensor-core prefill is off (GHOST_INFER_NO_TC_ATT, src/cuda.rs:5648-5654) or the head size has none
 * (src/cuda.rs:8452-8476). gi_attention / gi_attention_i8 take this path for prompts with bit 1 of exact set. */
int gi_attn_prefill_f32(void* stream, const void* q, int q_dtype, long long q_stride, const void* kc, const void* vc,
                        const float* ks, const float* vs, int kv_int8, long long kv_stride, long long kv_head_stride,
                        long long sc_stride, long long sc_head_stride, void* out, int out_dtype, long long out_stride,
                        int pos0, int n, int n_heads, int n_kv, int hd, float scale);

/* Bytes of the workspace gi_attn_prefill_i8_ws / gi_attn_prefill_q4_ws take for kv_len = pos0 + n keys (fmt 1: the
 * int8 cache, hd 64, 128 or 256; fmt 2: the 4-bit cache, hd 256); 0 for any other shape. No counterpart in the
 * reference, whose prefill widens each tile inside the kernel: f16 K and V rows [n_kv][kv_len][hd] (and for int8
 * f32 scales [n_kv][kv_len]), 256-byte aligned regions. */
size_t gi_attn_prefill_workspace_bytes(int kv_len, int n_kv, int hd, int fmt);

/* gi_attn_prefill_i8 / gi_attn_prefill_q4 with a caller-owned workspace (256-byte aligned, at least
 * gi_attn_prefill_workspace_bytes(pos0 + n, ...) bytes): the keys 0..pos0+n-1 are first widened into it to the f16
 * values the tiles take (int8: the exact integers, the scales kept apart; 4-bit: f16((n - 8) * scale)), and the
 * prefill then stages the widened tiles as it stages the f16 cache. The same arithmetic and outputs, bit for bit, as
 * the entry points without a workspace (replaces what they replace). gi_attention_i8 / gi_attention_q4 take this
 * path for prefill batches whenever their workspace holds it. */
int gi_attn_prefill_i8_ws(void* stream, const void* q, int q_dtype, long long q_stride, const int8_t* kc,
                          const int8_t* vc, const float* ks, const float* vs, long long kv_stride,
                          long long kv_head_stride, long long sc_stride, long long sc_head_stride, void* out,
                          int out_dtype, long long out_stride, int pos0, int n, int n_heads, int n_kv, int hd,
                          float scale, void* workspace, size_t workspace_bytes);
int gi_attn_prefill_q4_ws(void* stream, const void* q, int q_dtype, long long q_stride, const uint8_t* kc,
                          const uint8_t* vc, const uint16_t* ks, const uint16_t* vs, long long kv_stride,
                          long long kv_head_stride, long long sc_stride, long long sc_head_stride, void* out,
                          int out_dtype, long long out_stride, int pos0, int n, int n_heads, int n_kv, float scale,
                          void* workspace, size_t workspace_bytes);

/* The attention operator of one layer, as GpuModel::attention (src/cuda.rs:8448-8541) dispatches it:
 * qkv rows are [q (n_heads*hd) | k | v] f32 (stride n_heads*hd + 2*n_kv*hd, src/cuda.rs:1713), out rows
 * n_heads*hd f32. Batches of >= 16 tokens go to prefill; the rest, and every batch with bit 0 of `exact` set (a
 * verify batch, the reference's s.exact), to the split decode path in launches of at most 15 tokens
 * (SPLIT_MAX_BATCH, src/cuda.rs:119). Bit 1 of `exact` is the reference's GHOST_INFER_NO_TC_ATT
 * (src/cuda.rs:5648-5655): prefill batches take the f32 prefill (gi_attn_prefill_f32) at head sizes up to 128 over
 * the f16 and int8 caches and the split path elsewhere, and at head size 256 over the int8 cache the split path
 * computes in f32 precision instead of attention_decode_tc256's roundings. fixed_split
 * with posp: the grid is sized for ctx_cap (the session capacity), as max_splits does. scale is
 * 1/sqrt(hd) as in the reference. */
int gi_attention(void* stream, const float* qkv, const uint16_t* kc, const uint16_t* vc, float* out,
                 void* workspace, size_t workspace_bytes, int pos0, const int* posp, int ctx_cap, int n, int n_heads,
                 int n_kv, int hd, int exact);

/* gi_attention over the reference's int8 cache: kc / vc int8 [position][n_kv][hd] with f32 scales ks / vs
 * [position][n_kv], the operator's (kc, vc, ks, vs) tuple (src/cuda.rs:8448-8541 with KV8). */
int gi_attention_i8(void* stream, const float* qkv, const int8_t* kc, const int8_t* vc, const float* ks,
                    const float* vs, float* out, void* workspace, size_t workspace_bytes, int pos0, const int* posp,
                    int ctx_cap, int n, int n_heads, int n_kv, int hd, int exact);

/* gi_attention over the reference's 4-bit cache (head size 256): kc / vc [position][n_kv][128] bytes, ks / vs
 * [position][n_kv][8] f16 (src/cuda.rs:8448-8541 with KV4). q rows of qkv are the rotated queries that
 * gi_qk_norm_rope_q4 leaves; out holds rotated rows, which the layer turns back with gi_hadamard_rows
 * (src/cuda.rs:9765-9768). */
int gi_attention_q4(void* stream, const float* qkv, const uint8_t* kc, const uint8_t* vc, const uint16_t* ks,
                    const uint16_t* vs, float* out, void* workspace, size_t workspace_bytes, int pos0, const int* posp,
                    int ctx_cap, int n, int n_heads, int n_kv, int exact);

/* The attention output of a 4-bit cache rotated back: every 256-value segment of rows rows (width floats each,
 * a multiple of 256, row_stride apart) through the normalized Walsh-Hadamard transform, in place, stream-ordered.
 * Replaces: hadamard_rows with block 256 and no signs (src/cuda.rs:4675-4693) as the layer launches it after
 * attention over a 4-bit cache (src/cuda.rs:9765-9768). */
int gi_hadamard_rows(void* stream, float* x, long long row_stride, int rows, int width);

/* The layer's step before attention, for a batch of n tokens at positions pos0.. (posp: read from device
 * memory, graph replay). ctx_cap: positions the cache holds; rows at positions outside [0, ctx_cap) are not
 * stored (a device position cannot write past the cache). Required (>= n) with posp; 0 without posp means
 * pos0 + n, which the caller has checked. qkv: f32 rows [q (n_heads*hd) | k (n_kv*hd) | v (n_kv*hd)], updated in place:
 * each q and k head gets an RMSNorm (skipped when qn and kn are NULL: ss = sum of squares, x * rsqrt(ss/hd
 * + eps) * weight) and RoPE on its first rope_dim dims (pairs (i, i + rope_dim/2) when neox, else
 * (2i, 2i+1); angle = pos * base^(-2i/rope_dim) / ff[i], ff NULL = 1). The k and v heads are then stored
 * into the f16 caches (round to nearest even) in the layout of gi_attn_decode. hd 64, 128 or 256.
 * Replaces: qk_norm_rope with an f16 cache (src/cuda.rs:437-486, kv_store src/cuda.rs:312-362), launched
 * by layer_attn (src/cuda.rs:9706-9717). */
int gi_qk_norm_rope(void* stream, float* qkv, const float* qn, const float* kn, uint16_t* kc, uint16_t* vc,
                    long long kv_stride, long long kv_head_stride, int pos0, const int* posp, int ctx_cap, int n,
                    int n_heads, int n_kv, int hd, int rope_dim, float base, const float* ff, int neox, float eps);

/* gi_qk_norm_rope with an int8 cache (the layouts of gi_attn_decode_i8): each k and v row is quantised as it
 * is stored, dd = max|x| / 127, byte = round-to-nearest-even(x * (1/dd)) (0 when dd is 0), and dd goes to
 * ks / vs. Replaces: qk_norm_rope compiled with KV8 (kv_store, src/cuda.rs:333-339). */
int gi_qk_norm_rope_i8(void* stream, float* qkv, const float* qn, const float* kn, int8_t* kc, int8_t* vc, float* ks,
                       float* vs, long long kv_stride, long long kv_head_stride, long long sc_stride,
                       long long sc_head_stride, int pos0, const int* posp, int ctx_cap, int n, int n_heads, int n_kv,
                       int hd, int rope_dim, float base, const float* ff, int neox, float eps);

/* gi_qk_norm_rope storing into the 4-bit cache (head size 256; layouts as gi_attn_decode_q4). After RMSNorm and
 * RoPE every q and k head is rotated by the normalized 256-point Walsh-Hadamard transform (Sylvester order,
 * bit-identical to kv4_fwht) and written back rotated; a v head is rotated on its way into the cache. Each row
 * is then quantised per group of 32 values: dh = f16(max|x| / 7), q = clamp(rint(x / dh), -7, 7) (0 when dh is
 * 0), stored as q + 8 with dh as the group's scale. Replaces: qk_norm_rope compiled with KV4 (src/cuda.rs:437-486,
 * kv_store src/cuda.rs:340-357, kv4_fwht src/cuda.rs:242-256). */
int gi_qk_norm_rope_q4(void* stream, float* qkv, const float* qn, const float* kn, uint8_t* kc, uint8_t* vc,
                       uint16_t* ks, uint16_t* vs, long long kv_stride, long long kv_head_stride, long long sc_stride,
                       long long sc_head_stride, int pos0, const int* posp, int ctx_cap, int n, int n_heads, int n_kv,
                       int rope_dim, float base, const float* ff, int neox, float eps);

/* Cache growth: copies rows (position t < n_rows, kv head h < n_kv) of row_bytes bytes from one cache layout
 * to another, stream-ordered, allocating nothing. Strides are in bytes (src: t*src_stride +
 * h*src_head_stride). For a head-major cache [n_kv][cap][hd] growing to capacity cap2: src_stride =
 * dst_stride = row_bytes, src_head_stride = cap*row_bytes, dst_head_stride = cap2*row_bytes; the f32 scales
 * of an int8 cache move the same way with row_bytes = 4. Source and destination must not overlap. Replaces:
 * LayerCache::resize's copy of the first `keep` rows (src/cuda.rs:9962-9976), which the engine calls as a
 * session grows in CTX_STEP = 4096-position steps (src/cuda.rs:10410); with the reference's [position][n_kv]
 * layout that copy is contiguous, with the head-major one every row moves. */
int gi_kv_relayout(void* stream, const void* src, long long src_stride, long long src_head_stride, void* dst,
                   long long dst_stride, long long dst_head_stride, int n_rows, int n_kv, int row_bytes);

/* Per-kernel GPU time, for benchmarks. No counterpart in the reference. While on (process-wide), every
 * kernel the library launches outside graph capture is bracketed by a pair of HIP events on its stream.
 * Not for production use: each launch creates two events. */
int gi_kernel_timing(int on);

/* Total milliseconds and launch count of kernel kind `kernel` ("decode_partial", "decode_combine",
 * "prefill", "qk_norm_rope", "kv_relayout" or "hadamard_rows") recorded since the previous read of that kind; waits for the recorded events and
 * releases them. */
int gi_kernel_timing_read(const char* kernel, double* total_ms, int* launches);

#ifdef __cplusplus
}
#endif

#endif /* GI_ATTN_H */
