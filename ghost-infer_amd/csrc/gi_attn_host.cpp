// C-ABI host side of the gfx950 attention path (declarations and contracts in include/gi_attn.h).
//
// Replaces the reference's NVRTC launch layer (src/cuda.rs:4870-5128 driver/NVRTC loading,
// src/cuda.rs:5377-5763 Kernels/launch3): the kernels are an offline-built code object loaded with
// hipModuleLoad once per device and launched by name with hipModuleLaunchKernel on the caller's stream.
// No entry point allocates device memory or synchronises the host.
#include "gi_attn.h"

#include <hip/hip_runtime.h>

#include <dlfcn.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

namespace {

// Must match the kernels' GiDecodeArgs (gi_attn_kernels.hip).
struct GiDecodeArgs {
    const float* q;
    const uint16_t* kc;
    const uint16_t* vc;
    float* part;
    float* out;
    const int* posp;
    long long q_stride;
    long long kv_stride;
    long long out_stride;
    long long kv_head_stride;
    int pos0;
    int n_tok;
    int n_heads;
    int n_kv;
    int chunk;
    int nsplit;
    float qscale;
    int hd;
    const float* ks;
    const float* vs;
    long long sc_stride;
    long long sc_head_stride;
    int kv_cap;
    int pad_;
};

// Must match the kernels' GiRopeArgs.
struct GiRopeArgs {
    float* qkv;
    const float* qn;
    const float* kn;
    uint16_t* kc;
    uint16_t* vc;
    const float* ff;
    const int* posp;
    long long row_stride;
    long long kv_stride;
    long long kv_head_stride;
    int pos0;
    int n;
    int n_heads;
    int n_kv;
    int hd;
    int rope_dim;
    float base;
    float eps;
    int neox;
    int fmt; // 0 f16, 1 int8, 2 the 4-bit cache
    float* ks;
    float* vs;
    long long sc_stride;
    long long sc_head_stride;
    int ctx_cap;
    int pad_;
};

// Must match the kernels' GiHadamardArgs.
struct GiHadamardArgs {
    float* x;
    long long row_stride;
    int rows;
    int segs;
};

// Must match the kernels' GiRelayoutArgs.
struct GiRelayoutArgs {
    const void* src;
    void* dst;
    long long src_stride;
    long long src_head_stride;
    long long dst_stride;
    long long dst_head_stride;
    long long n_units;
    int n_rows;
    int units_per_row;
    int unit;
    int pad_;
};

// Must match the kernels' GiWidenArgs.
struct GiWidenArgs {
    const void* kc;
    const void* vc;
    const void* ks;
    const void* vs;
    void* kw;
    void* vw;
    float* ksw;
    float* vsw;
    long long kv_stride;
    long long kv_head_stride;
    long long sc_stride;
    long long sc_head_stride;
    int n_rows;
    int n_kv;
    int hd;
    int fmt;
    float vbias;
    int pad_;
};
constexpr float kPrefillI8VBias = 8.f; // the head-64/128 int8 prefill's value-scale bias (the kernels' PF_I8_VBIAS)

// Must match the kernels' GiPrefillArgs.
struct GiPrefillArgs {
    const void* q;
    const uint16_t* kc;
    const uint16_t* vc;
    void* out;
    long long q_stride;
    long long kv_stride;
    long long out_stride;
    long long kv_head_stride;
    int pos0;
    int n;
    int n_heads;
    int n_kv;
    float qscale;
    int q_f16;
    int out_f16;
    int hd;
    const float* ks;
    const float* vs;
    long long sc_stride;
    long long sc_head_stride;
};

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kF32Rows = 128;   // query rows per gi_prefill_f32_* workgroup; must match the kernels' PF32_ROWS
constexpr int kF32Threads = 512; // its block size (8 waves of 16 rows)

// Head sizes of the f32 kernels (gi_attn_f32.hip): the multiples of 16 up to 112 that the MFMA kernels do not
// take, the reference's f32 fallback cases (attention_partial / attention_prefill, src/cuda.rs:1866-2041).
bool f32_hd(int hd) { return hd % 16 == 0 && hd >= 16 && hd <= 112 && hd != 64; }
constexpr int kF32Sizes[6] = {16, 32, 48, 80, 96, 112}; // the f32 kernels' builds, in this order
int f32_index(int hd) { return hd < 64 ? hd / 16 - 1 : hd / 16 - 2; }
constexpr int kMaxDevices = 64;
constexpr int kRopeHeads = 16; // heads per gi_qk_norm_rope workgroup; must match the kernels' ROPE_HEADS
constexpr int kCombineSplit = 8; // combine workgroups per (head, token); must match the kernels' CMB_DSPLIT
constexpr int kDecWaves = 4, kDecTile = 32, kDecPairs = 8; // slice partials are hd + 4 floats
constexpr int kSliceUnit = kDecWaves * kDecTile; // 128 keys
constexpr int kSplitMaxBatch = 15;                // tokens per split launch (src/cuda.rs:119)
constexpr int kTiledMinBatch = 16;                // prefill from this many tokens (src/cuda.rs:95)
constexpr int kPrefillRows = 256; // query rows per prefill workgroup; must match the kernels' PF_BQ
constexpr int kPrefill256rRows = 128; // the same for gi_prefill_fwd_h256r (PF256R_BQ)

thread_local std::string g_err;

int fail(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return GI_EINVAL;
}

int check(hipError_t r, const char* what) {
    if (r == hipSuccess) return 0;
    char buf[512];
    snprintf(buf, sizeof buf, "HIP %s failed: %s (%d)", what, hipGetErrorString(r), (int)r);
    g_err = buf;
    return (int)r;
}

struct Module {
    bool loaded = false;
    hipModule_t mod = nullptr;
    hipFunction_t dec[2] = {};        // up to 8 pairs, head size 128: [int8 cache]
    // one-buffer forms for slices of at most two tiles per wave: f16, int8, f16 hd 64, f16 hd 256, int8 hd 256, 4-bit
    hipFunction_t dec_short[6] = {};
    hipFunction_t dec256 = nullptr;   // up to 8 pairs, head size 256, the f16 cache
    hipFunction_t dec64[2][3] = {};   // head size 64: [int8 cache][up to 8 pairs, one column block, two]
    hipFunction_t dec_pm[2][2] = {};  // [int8 cache][column blocks - 1]: one pair per column
    hipFunction_t dec_ws2[2] = {};    // head size 128, two column blocks, two pair sets of two waves: [int8 cache]
    hipFunction_t dec_ref[3] = {};    // head size 256, one pair per column, the reference's tc256 roundings: int8
                                      // one column block, 4-bit one and two column blocks
    hipFunction_t dec_pm256[2] = {};  // head size 256, one pair per column, two pair sets of two waves: [f16, int8]
    hipFunction_t dec_i8_256f[2] = {}; // head size 256 over the int8 cache in f32 precision: [up to 8 pairs, above]
    hipFunction_t prefill[2] = {};   // [int8 cache], head size 128
    hipFunction_t prefill64[2] = {}; // [int8 cache], head size 64 (the same launch shape and block size)
    hipFunction_t dec_f32[2][6] = {}, prefill_f32[2][6] = {}; // the f32 kernels: [int8 cache][kF32Sizes index]
    hipFunction_t prefill_f32p[2][2] = {}; // f32 prompts at head sizes 64 and 128: [int8 cache][64, 128]
    hipFunction_t prefill256r = nullptr; // head size 256 (f16 cache), 16 rows per wave: one workgroup per query tile
    hipFunction_t prefill256r_fmt[2] = {}; // the same over the int8 and the 4-bit cache
    // pre-widened staging: gi_kv_widen, then the int8 kernels that stage the widened tiles by LDS-DMA (head sizes
    // 128, 64, 256; the widened 4-bit cache runs prefill256r)
    hipFunction_t widen = nullptr, prefill_i8s[3] = {};
    hipFunction_t combine = nullptr, rope = nullptr, relayout = nullptr, hadamard = nullptr;
    int prefill_threads[2] = {}; // each prefill kernel's block size (its launch bound: waves x 64)
    int prefill256r_threads = 0;
    // gi_attn_decode_noalloc's partials: the device address of the code object's gi_scratch array on this
    // device (the array's host-side name is no device address; the module gives the real one at load)
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
};
std::mutex g_mu;
Module g_mods[kMaxDevices];

// The code object: $GI_CODE_OBJECT when set, else gi_attn_gfx950.hsaco beside this library.
std::string default_code_object() {
    if (const char* env = getenv("GI_CODE_OBJECT"))
        if (*env) return env;
    Dl_info info;
    if (dladdr((void*)&default_code_object, &info) && info.dli_fname) {
        std::string p = info.dli_fname;
        size_t slash = p.rfind('/');
        return (slash == std::string::npos ? std::string(".") : p.substr(0, slash)) + "/gi_attn_gfx950.hsaco";
    }
    return "gi_attn_gfx950.hsaco";
}

int load_module(const char* path, Module** out) {
    int dev = 0;
    if (int e = check(hipGetDevice(&dev), "hipGetDevice")) return e;
    if (dev < 0 || dev >= kMaxDevices) return fail("device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_mu);
    Module& m = g_mods[dev];
    if (!m.loaded) {
        std::string p = path ? std::string(path) : default_code_object();
        if (int e = check(hipModuleLoad(&m.mod, p.c_str()), ("hipModuleLoad(" + p + ")").c_str())) return e;
        struct { hipFunction_t* f; const char* name; } fns[] = {
            {&m.dec[0], "gi_decode_partial_1"},
            {&m.dec_short[0], "gi_decode_partial_1s"},
            {&m.dec_short[1], "gi_decode_partial_1s_i8"},
            {&m.dec_short[2], "gi_decode_partial_1s_h64"},
            {&m.dec_short[3], "gi_decode_partial_1s_h256"},
            {&m.dec_short[4], "gi_decode_pm_1s_i8_h256"},
            {&m.dec_short[5], "gi_decode_pm_1s_q4"},
            {&m.dec[1], "gi_decode_partial_1_i8"},
            {&m.dec256, "gi_decode_partial_1_h256"},
            {&m.dec64[0][0], "gi_decode_partial_1_h64"},
            {&m.dec64[0][1], "gi_decode_pm_1_h64"},
            {&m.dec64[0][2], "gi_decode_pm_2_h64"},
            {&m.dec64[1][0], "gi_decode_partial_1_i8_h64"},
            {&m.dec64[1][1], "gi_decode_pm_1_i8_h64"},
            {&m.dec64[1][2], "gi_decode_pm_2_i8_h64"},
            {&m.dec_ref[0], "gi_decode_pm_1_i8_h256"},
            {&m.dec_ref[1], "gi_decode_pm_1_q4"},
            {&m.dec_ref[2], "gi_decode_pm_2_q4"},
            {&m.dec_pm[0][0], "gi_decode_pm_1"},
            {&m.dec_pm[0][1], "gi_decode_pm_2"},
            {&m.dec_pm[1][0], "gi_decode_pm_1_i8"},
            {&m.dec_pm[1][1], "gi_decode_pm_2_i8"},
            {&m.dec_ws2[0], "gi_decode_pm_ws2_2"},
            {&m.dec_ws2[1], "gi_decode_pm_ws2_2_i8"},
            {&m.dec_pm256[0], "gi_decode_pm_ws2_1_h256"},
            {&m.dec_pm256[1], "gi_decode_pm_ws2_1_i8_h256"},
            {&m.dec_i8_256f[0], "gi_decode_partial_1_i8_h256f"},
            {&m.dec_i8_256f[1], "gi_decode_pm_ws2_1_i8_h256f"},
            {&m.combine, "gi_decode_combine"},
            {&m.relayout, "gi_kv_relayout"},
            {&m.hadamard, "gi_hadamard_rows"},
            {&m.prefill[0], "gi_prefill_fwd"},
            {&m.prefill[1], "gi_prefill_fwd_i8"},
            {&m.prefill64[0], "gi_prefill_fwd_h64"},
            {&m.prefill64[1], "gi_prefill_fwd_h64_i8"},
            {&m.prefill256r, "gi_prefill_fwd_h256r"},
            {&m.prefill256r_fmt[0], "gi_prefill_fwd_h256r_i8"},
            {&m.prefill256r_fmt[1], "gi_prefill_fwd_h256r_q4"},
            {&m.widen, "gi_kv_widen"},
            {&m.prefill_i8s[0], "gi_prefill_fwd_i8s"},
            {&m.prefill_i8s[1], "gi_prefill_fwd_h64_i8s"},
            {&m.prefill_i8s[2], "gi_prefill_fwd_h256r_i8s"},
            {&m.rope, "gi_qk_norm_rope"},
        };
        for (auto& f : fns)
            if (int e = check(hipModuleGetFunction(f.f, m.mod, f.name), f.name)) {
                (void)hipModuleUnload(m.mod);
                m.mod = nullptr;
                return e;
            }
        for (int i8 = 0; i8 < 2; i8++)
            for (int i = 0; i < 6; i++) {
                char dn[64], pn[64];
                snprintf(dn, sizeof dn, "gi_decode_f32%s_h%d", i8 ? "_i8" : "", kF32Sizes[i]);
                snprintf(pn, sizeof pn, "gi_prefill_f32%s_h%d", i8 ? "_i8" : "", kF32Sizes[i]);
                int e = check(hipModuleGetFunction(&m.dec_f32[i8][i], m.mod, dn), dn);
                if (!e) e = check(hipModuleGetFunction(&m.prefill_f32[i8][i], m.mod, pn), pn);
                if (!e && i < 2) {
                    snprintf(pn, sizeof pn, "gi_prefill_f32%s_h%d", i8 ? "_i8" : "", 64 << i);
                    e = check(hipModuleGetFunction(&m.prefill_f32p[i8][i], m.mod, pn), pn);
                }
                if (e) {
                    (void)hipModuleUnload(m.mod);
                    m.mod = nullptr;
                    return e;
                }
            }
        if (int e = check(hipFuncGetAttribute(&m.prefill_threads[0], HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, m.prefill[0]),
                          "hipFuncGetAttribute(gi_prefill_fwd)") ||
                    check(hipFuncGetAttribute(&m.prefill_threads[1], HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, m.prefill[1]),
                          "hipFuncGetAttribute(gi_prefill_fwd_i8)") ||
                    check(hipFuncGetAttribute(&m.prefill256r_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK,
                                              m.prefill256r),
                          "hipFuncGetAttribute(gi_prefill_fwd_h256r)")) {
            (void)hipModuleUnload(m.mod);
            m.mod = nullptr;
            return e;
        }
        hipDeviceptr_t sp = nullptr;
        if (int e = check(hipModuleGetGlobal(&sp, &m.scratch_bytes, m.mod, "gi_scratch"), "hipModuleGetGlobal(gi_scratch)")) {
            (void)hipModuleUnload(m.mod);
            m.mod = nullptr;
            return e;
        }
        m.scratch = (void*)sp;
        m.loaded = true;
    }
    *out = &m;
    return 0;
}

// ---- per-kernel timing (gi_kernel_timing): event pairs around each launch, per kernel kind
enum Kind { kDecodePartial = 0, kDecodeCombine = 1, kPrefill = 2, kRope = 3, kRelayout = 4, kHadamard = 5, kWiden = 6,
            kKinds = 7 };
const char* const kKindNames[kKinds] = {"decode_partial", "decode_combine", "prefill", "qk_norm_rope", "kv_relayout",
                                        "hadamard_rows", "kv_widen"};
struct Timing {
    std::mutex mu;
    bool on = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> ev[kKinds];
};
Timing g_timing;

int launch(Kind kind, hipFunction_t f, dim3 grid, dim3 block, hipStream_t stream, void* args, size_t args_size) {
    void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &args_size,
                      HIP_LAUNCH_PARAM_END};
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (g_timing.on) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) {
            // timing-only events: no system-scope fence (cache writeback/invalidate) around the kernel
            if (int e = check(hipEventCreateWithFlags(&e0, hipEventDisableSystemFence), "hipEventCreate")) return e;
            if (int e = check(hipEventCreateWithFlags(&e1, hipEventDisableSystemFence), "hipEventCreate")) return e;
            if (int e = check(hipEventRecord(e0, stream), "hipEventRecord")) return e;
        }
    }
    int r = check(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, 0, stream, nullptr,
                                        config),
                  "kernel launch");
    if (e0) {
        if (int e = check(hipEventRecord(e1, stream), "hipEventRecord")) return e;
        std::lock_guard<std::mutex> lock(g_timing.mu);
        g_timing.ev[kind].emplace_back(e0, e1);
    }
    return r;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Workgroups to aim for per decode launch: one per CU of the 256 on MI355X. A decode workgroup holds a
// whole CU's registers, so more workgroups run in sequential rounds, each paying the ramp-up and drain of
// the memory pipeline.
int decode_target_wgs() {
    static int target = [] {
        const char* e = getenv("GI_DECODE_TARGET_WGS");
        int v = e ? atoi(e) : 0;
        return v > 0 ? v : 256;
    }();
    return target;
}

// Decode kernel variant for n_tok tokens of G heads per kv head (head size hd, cache format fmt: 0 f16, 1 int8,
// 2 4-bit). Up to 8 (token, head) pairs: one column block of 8 pairs, each pair's f16 high and remainder parts in
// two columns (gi_decode_partial_1). More pairs: one pair per column (pm), 16 per column block, the high and
// remainder parts as two MFMAs into one accumulator, so no lane repeats its neighbour's softmax. Head size 256 over
// the int8 and 4-bit caches: one pair per column with the reference's single f16 Q and P, 16 pairs per workgroup
// up to 16 pairs, else two column blocks per wave (32 pairs per workgroup), each tile widened once per workgroup.
struct DecVariant {
    int ncb;     // column blocks per wave
    bool ws2;    // two pair sets per workgroup, each split over two waves (else the 4 waves serve one set)
    bool pm;     // one pair per column
    int groups;  // workgroups per (slice, kv head)
};
DecVariant dec_variant(int n_tok, int G, int hd = 128, int fmt = 0) {
    const int pairs = n_tok * G;
    const bool i8 = fmt == 1;
    if (f32_hd(hd)) return DecVariant{1, false, false, 1}; // one workgroup per (slice, head, token)
    if (hd == 256 && fmt) {
        // Above 16 pairs, split kernel at 32768 keys, 64 pairs, 16/2 (same box): 4-bit two column blocks per wave
        // 29.0 us, two pair sets of one block over two waves each 29.5 (the hi/lo-split kernel before: 31.3); int8
        // 52.3 and 25.4 (before: 28.4; two column blocks leave room for two tiles in flight, not four)
        if (pairs <= 2 * kDecPairs) return DecVariant{1, false, true, 1};
        if (fmt == 1) return DecVariant{1, true, true, (pairs + 4 * kDecPairs - 1) / (4 * kDecPairs)};
        return DecVariant{2, false, true, (pairs + 4 * kDecPairs - 1) / (4 * kDecPairs)};
    }
    DecVariant v{1, false, pairs > kDecPairs, 1};
    if (!v.pm) return v;
    if (hd == 64) {
        // one pair per column: one column block up to 16 pairs, else two per wave (32 pairs per workgroup)
        v.ncb = pairs > 2 * kDecPairs ? 2 : 1;
        v.groups = (pairs + 2 * kDecPairs * v.ncb - 1) / (2 * kDecPairs * v.ncb);
        return v;
    }
    if (hd == 256) {
        // two pair sets of 16 per workgroup, each over two waves that split the slice's tiles (two column
        // blocks per wave exceed the register file at this head size). Split kernel at 32768 keys, 16/2, against
        // 4 waves of 16 pairs each walking every tile (which beat the hi/lo column layout at 16-128 pairs):
        // f16 16 pairs 20.2 -> 17.1 us, 24 pairs 22.7 -> 23.4, 64 pairs 37.9 -> 34.6, 128 pairs 58.4 -> 55.5;
        // int8 26.0 -> 18.3, 28.1 -> 20.9, 34.4 -> 30.4, 51.9 -> 47.7; 4-bit 30.9 -> 20.2, 32.9 -> 23.2,
        // 40.3 -> 35.0, 60.2 -> 53.9.
        v.ws2 = true;
        v.groups = (pairs + 4 * kDecPairs - 1) / (4 * kDecPairs);
        return v;
    }
    // head size 128, above 16 pairs: two column blocks per wave, each wave on slice tiles of its own, and as
    // many pair groups (workgroups per (slice, kv head), placed on one XCD) as needed: every tile is loaded,
    // transposed and masked once per workgroup, and each wave has two independent MFMA chains. Measured
    // against 4 waves sharing every tile: config 4's 64 pairs 32.5 -> 27.8 us (f16), 32.5 -> 28.4 us
    // (int8); 96 pairs 36.5 -> 34.3 and 50.1 -> 35.5 us; equal at 48 and 128 pairs (f16).
    v.ncb = pairs > 2 * kDecPairs ? 2 : 1;
    // int8 (on the pipelined tile loop) takes the same layout where its pair groups of 64 are full, measured
    // at 32768 keys, 32/4 (step µs): 128 pairs 39.9 -> 39.1, 256 pairs 63.1 -> 60.5; at 64 pairs 27.7 ->
    // 28.0, and at 80 and 96 pairs (a second group part empty) 33.5 -> 36.8 and 34.0 -> 37.0.
    if (!i8 ? pairs > 4 * kDecPairs : pairs > 8 * kDecPairs && pairs % (8 * kDecPairs) == 0) {
        // f16 above 32 pairs: two pair sets of 32 per workgroup, each split over two waves, so a tile's second
        // read comes from the same CU rather than another workgroup. Split kernel at 32768 keys, 32/4:
        // 48 pairs 27.1 -> 25.9 us, 64 pairs 27.9 -> 26.9, 96 pairs 34.6 -> 34.2, 128 pairs 40.7 -> 37.2.
        // The int8 cache lost at 64 pairs (28.0 -> 31.2 us, before its pipelined loop): its tiles are half the
        // bytes, so the read that moves is cheap while the halved waves per pair set lengthen the chain.
        v.ws2 = true;
        v.groups = (pairs + 8 * kDecPairs - 1) / (8 * kDecPairs);
        return v;
    }
    v.groups = (pairs + 2 * kDecPairs * v.ncb - 1) / (2 * kDecPairs * v.ncb);
    return v;
}

// Most slices per (kv head, pair group): the grid stays near decode_target_wgs() workgroups. The f32 kernels take
// one workgroup per (slice, head) and hold few registers, so they aim at four workgroups per CU.
int slices_per_slot(int n_heads, int n_kv, int groups, int hd) {
    if (f32_hd(hd)) return std::max(1, 4 * decode_target_wgs() / std::max(1, n_heads));
    return std::max(1, decode_target_wgs() / std::max(1, n_kv * groups));
}

// Slices of a span: at most per_slot per (kv head, pair group), so the grid stays near decode_target_wgs(). A
// slice holds whole wave tiles (unit / 4 keys: the waves of a workgroup take a slice's tiles in turn) and at least
// `unit` keys (one tile per wave), and is as short as the cap allows: within one tile of the span's even share
// over per_slot slices. At config 4's 32776 keys: 61 slices of 544 keys, where whole units of 4 tiles gave 52
// slices of 640 (208 of 256 workgroups busy).
void plan(int max_span, int n_tok, int n_heads, int n_kv, int* chunk, int* nsplit, int unit = kSliceUnit,
          int hd = 128, int fmt = 0) {
    int G = n_heads / n_kv;
    int groups = dec_variant(n_tok, G, hd, fmt).groups;
    int per_slot = slices_per_slot(n_heads, n_kv, groups, hd);
    const int tile = unit / kDecWaves;
    const int least = (max_span + per_slot - 1) / per_slot; // the shortest slice the cap allows
    *chunk = std::max(unit, (least + tile - 1) / tile * tile);
    *nsplit = std::max(1, (max_span + *chunk - 1) / *chunk);
}

// K/V rows of hd elements must not overlap: either positions outer (kv_stride covers all heads) or heads
// outer (a head's block holds whole rows); both strides in 16-byte units (`unit` elements: 8 f16, 16 int8).
int check_kv_strides(long long kv_stride, long long kv_head_stride, int n_kv, int hd, int unit = 8) {
    if (kv_stride % unit || kv_head_stride % unit || kv_stride <= 0 || kv_head_stride <= 0)
        return fail("kv_stride %lld and kv_head_stride %lld must be positive multiples of %d", kv_stride, kv_head_stride,
                    unit);
    bool pos_outer = kv_head_stride >= hd && kv_stride >= (long long)n_kv * kv_head_stride;
    bool head_outer = kv_stride >= hd && (n_kv == 1 || kv_head_stride >= kv_stride);
    if (!pos_outer && !head_outer)
        return fail("kv_stride %lld / kv_head_stride %lld overlap rows of %d kv heads", kv_stride, kv_head_stride, n_kv);
    return 0;
}

// An int8 cache's scales: positive strides (in floats), 4-byte aligned arrays.
int check_scales(const float* ks, const float* vs, long long sc_stride, long long sc_head_stride) {
    if (!ks || !vs) return fail("null scale pointer");
    if (((uintptr_t)ks & 3) || ((uintptr_t)vs & 3)) return fail("ks and vs must be 4-byte aligned");
    if (sc_stride <= 0 || sc_head_stride <= 0)
        return fail("sc_stride %lld and sc_head_stride %lld must be positive", sc_stride, sc_head_stride);
    return 0;
}

// Keys per slice unit: one tile per wave (32 f16 keys at head size 128, 64 int8 keys, 16 f16 keys at 256).
int slice_unit(bool i8, int hd) { return hd == 256 ? kDecWaves * kDecTile / 2 : i8 ? 2 * kSliceUnit : kSliceUnit; }

// Head sizes 64 (attn_prefill_tc<64>, src/cuda.rs:2620; attention_partial_gqa at any multiple of 32), 128 and 256
// on the MFMA kernels (the 4-bit cache: 256 only, checked by its entry points), and the f32 kernels' multiples of
// 16 up to 112.
int check_shape(int n_heads, int n_kv, int hd, bool = true) {
    if (hd != 64 && hd != 128 && hd != 256 && !f32_hd(hd))
        return fail("head size %d unsupported (the gfx950 kernels take 64, 128, 256 and the multiples of 16 up to "
                    "112)", hd);
    if (n_kv <= 0 || n_heads <= 0 || n_heads % n_kv != 0)
        return fail("n_heads %d must be a positive multiple of n_kv %d", n_heads, n_kv);
    return 0;
}

// gi_attn_decode, gi_attn_decode_i8 and gi_attn_decode_q4: the same launch with the f16, int8 or 4-bit kernels
// (fmt 0, 1, 2).
int decode_impl(void* stream, const float* q, long long q_stride, const void* kc, const void* vc, const float* ks,
                const float* vs, long long sc_stride, long long sc_head_stride, int fmt, long long kv_stride,
                long long kv_head_stride, float* out, long long out_stride, void* workspace, size_t workspace_bytes,
                int pos0, const int* posp, int ctx_cap, int n_tok, int n_heads, int n_kv, int hd, float scale,
                bool f32_256 = false) {
    if (int e = check_shape(n_heads, n_kv, hd, true)) return e;
    if (fmt == 2 && hd != 256) return fail("the 4-bit cache takes head size 256 only (got %d)", hd);
    const bool i8 = fmt == 1;
    if (n_tok <= 0) return fail("n_tok %d must be positive", n_tok);
    if (!q || !kc || !vc || !out) return fail("null tensor pointer");
    if (fmt == 2) {
        // rows of 128 bytes (kv strides in bytes), 8 f16 scales a row (scale strides in f16 elements)
        if (kv_head_stride == 0) kv_head_stride = hd / 2;
        if (int e = check_kv_strides(kv_stride, kv_head_stride, n_kv, hd / 2, 16)) return e;
        if (!ks || !vs) return fail("null scale pointer");
        // (the kernels read a row's scales in 4-byte words)
        if (((uintptr_t)ks & 3) || ((uintptr_t)vs & 3) || ((sc_stride | sc_head_stride) & 1))
            return fail("ks and vs must be 4-byte aligned and their strides even");
        if (int e = check_kv_strides(sc_stride, sc_head_stride, n_kv, 8, 1)) return e;
    } else {
        if (kv_head_stride == 0) kv_head_stride = hd;
        if (int e = check_kv_strides(kv_stride, kv_head_stride, n_kv, hd, fmt ? 16 : 8)) return e;
        if (fmt)
            if (int e = check_scales(ks, vs, sc_stride, sc_head_stride)) return e;
    }
    if (!aligned16(q) || !aligned16(kc) || !aligned16(vc) || q_stride % 4)
        return fail("q, kc, vc must be 16-byte aligned and q_stride a multiple of 4");
    if (q_stride < (long long)n_heads * hd || out_stride < (long long)n_heads * hd)
        return fail("row strides too small for %d heads", n_heads);
    if (!posp && pos0 < 0) return fail("pos0 %d must be >= 0", pos0);
    int max_span = posp ? ctx_cap : pos0 + n_tok;
    if (posp && ctx_cap < n_tok) return fail("ctx_cap %d must cover the %d tokens", ctx_cap, n_tok);
    Module* m;
    if (int e = load_module(nullptr, &m)) return e;
    // f32_256: head size 256 over the int8 cache in f32 precision, with the f16 cache's pair layouts and slice plan
    const bool f32_i8 = f32_256 && fmt == 1 && hd == 256;
    const int vfmt = f32_i8 ? 0 : fmt;
    const DecVariant var = dec_variant(n_tok, n_heads / n_kv, hd, vfmt);
    GiDecodeArgs a{};
    plan(max_span, n_tok, n_heads, n_kv, &a.chunk, &a.nsplit, slice_unit(i8, hd), hd, vfmt);
    size_t need = a.nsplit == 1 ? 0 : (size_t)n_tok * n_heads * a.nsplit * (hd + 4) * sizeof(float);
    if (need && (!workspace || workspace_bytes < need))
        return fail("workspace of %zu bytes too small: %zu needed", workspace_bytes, need);
    if (need && !aligned16(workspace)) return fail("the workspace must be 16-byte aligned");
    a.q = q;
    a.kc = (const uint16_t*)kc;
    a.vc = (const uint16_t*)vc;
    a.part = (float*)workspace;
    a.kv_cap = posp ? ctx_cap : pos0 + n_tok;
    a.out = out;
    a.posp = posp;
    a.q_stride = q_stride;
    a.kv_stride = kv_stride;
    a.out_stride = out_stride;
    a.kv_head_stride = kv_head_stride;
    a.pos0 = pos0;
    a.n_tok = n_tok;
    a.n_heads = n_heads;
    a.n_kv = n_kv;
    a.qscale = scale * kLog2e;
    a.hd = hd;
    if (fmt) {
        a.ks = ks;
        a.vs = vs;
        a.sc_stride = sc_stride;
        a.sc_head_stride = sc_head_stride;
    }
    hipStream_t st = (hipStream_t)stream;
    if (f32_hd(hd)) {
        if (int e = launch(kDecodePartial, m->dec_f32[i8][f32_index(hd)], dim3(a.nsplit, n_heads, n_tok), dim3(256), st, &a, sizeof a))
            return e;
        if (a.nsplit == 1) return 0;
        return launch(kDecodeCombine, m->combine, dim3(n_heads, n_tok, kCombineSplit * hd / 128), dim3(64), st, &a,
                      sizeof a);
    }
    hipFunction_t f = f32_i8      ? m->dec_i8_256f[var.ws2 ? 1 : 0]
                      : hd == 64  ? m->dec64[i8][var.pm ? var.ncb : 0]
                      : hd == 256 ? (var.ws2 ? m->dec_pm256[fmt] : fmt ? m->dec_ref[fmt - 1 + var.ncb - 1]
                                   : var.pm ? m->dec_pm256[0] : m->dec256)
                      : var.ws2   ? m->dec_ws2[i8]
                      : var.pm    ? m->dec_pm[i8][var.ncb - 1]
                                  : m->dec[i8];
    // slices of at most two tiles per wave (kDecWaves waves of kDecTile keys each): the one-buffer kernel
    if (f == m->dec[0] && a.chunk <= 2 * kDecWaves * kDecTile) f = m->dec_short[0];
    else if (f == m->dec[1] && a.chunk <= 4 * kDecWaves * kDecTile) f = m->dec_short[1]; // (int8 tiles: 64 keys)
    else if (f == m->dec64[0][0] && a.chunk <= 2 * kDecWaves * kDecTile) f = m->dec_short[2];
    else if (a.chunk <= kDecWaves * kDecTile) { // head size 256 (16-key tiles)
        if (f == m->dec256) f = m->dec_short[3];
        else if (f == m->dec_ref[0]) f = m->dec_short[4];
        else if (f == m->dec_ref[1]) f = m->dec_short[5];
    }
    if (int e = launch(kDecodePartial, f, dim3(a.nsplit, n_kv, var.groups), dim3(256), st, &a, sizeof a)) return e;
    if (a.nsplit == 1) return 0;
    return launch(kDecodeCombine, m->combine, dim3(n_heads, n_tok, kCombineSplit * hd / 128), dim3(64), st, &a, sizeof a);
}

// gi_qk_norm_rope, gi_qk_norm_rope_i8 and gi_qk_norm_rope_q4: one kernel; fmt 0 f16, 1 int8, 2 the 4-bit cache.
int rope_impl(void* stream, float* qkv, const float* qn, const float* kn, void* kc, void* vc, float* ks, float* vs,
              long long sc_stride, long long sc_head_stride, int fmt, long long kv_stride, long long kv_head_stride,
              int pos0, const int* posp, int ctx_cap, int n, int n_heads, int n_kv, int hd, int rope_dim, float base,
              const float* ff, int neox, float eps) {
    if (fmt == 2 && hd != 256) return fail("the 4-bit cache takes head size 256 only (got %d)", hd);
    if (hd != 64 && hd != 128 && hd != 256 && !f32_hd(hd))
        return fail("head size %d unsupported by the KV store (64, 128, 256, the multiples of 16 up to 112)", hd);
    if (n_kv <= 0 || n_heads <= 0 || n_heads % n_kv != 0)
        return fail("n_heads %d must be a positive multiple of n_kv %d", n_heads, n_kv);
    if (n <= 0) return fail("n %d must be positive", n);
    if (rope_dim < 0 || rope_dim > hd || rope_dim % 2) return fail("rope_dim %d must be even and at most %d", rope_dim, hd);
    if (!qkv || !kc || !vc) return fail("null tensor pointer");
    if ((qn == nullptr) != (kn == nullptr)) return fail("qn and kn must both be given or both be null");
    if (!posp && pos0 < 0) return fail("pos0 %d must be >= 0", pos0);
    if (posp && ctx_cap < n) return fail("with posp, ctx_cap %d must cover the %d tokens", ctx_cap, n);
    if (!posp && ctx_cap > 0 && ctx_cap < pos0 + n)
        return fail("positions %d..%d exceed ctx_cap %d", pos0, pos0 + n - 1, ctx_cap);
    if (fmt == 2) {
        // rows of 128 bytes (kv strides in bytes), 8 f16 scales a row (scale strides in f16 elements)
        if (kv_head_stride == 0) kv_head_stride = hd / 2;
        if (int e = check_kv_strides(kv_stride, kv_head_stride, n_kv, hd / 2, 16)) return e;
        if (!ks || !vs) return fail("null scale pointer");
        if (((uintptr_t)ks & 1) || ((uintptr_t)vs & 1)) return fail("ks and vs must be 2-byte aligned");
        if (int e = check_kv_strides(sc_stride, sc_head_stride, n_kv, 8, 1)) return e;
    } else {
        if (kv_head_stride == 0) kv_head_stride = hd;
        if (int e = check_kv_strides(kv_stride, kv_head_stride, n_kv, hd, fmt ? 16 : 8)) return e;
        if (fmt)
            if (int e = check_scales(ks, vs, sc_stride, sc_head_stride)) return e;
    }
    Module* m;
    if (int e = load_module(nullptr, &m)) return e;
    GiRopeArgs a{};
    a.ctx_cap = ctx_cap > 0 ? ctx_cap : pos0 + n;
    a.qkv = qkv;
    a.qn = qn;
    a.kn = kn;
    a.kc = (uint16_t*)kc;
    a.vc = (uint16_t*)vc;
    a.fmt = fmt;
    a.ks = ks;
    a.vs = vs;
    a.sc_stride = sc_stride;
    a.sc_head_stride = sc_head_stride;
    a.ff = ff;
    a.posp = posp;
    a.row_stride = (long long)(n_heads + 2 * n_kv) * hd;
    a.kv_stride = kv_stride;
    a.kv_head_stride = kv_head_stride;
    a.pos0 = pos0;
    a.n = n;
    a.n_heads = n_heads;
    a.n_kv = n_kv;
    a.hd = hd;
    a.rope_dim = rope_dim;
    a.base = base;
    a.eps = eps;
    a.neox = neox != 0;
    const int groups = (n_heads + 2 * n_kv + kRopeHeads - 1) / kRopeHeads; // workgroups per token
    return launch(kRope, m->rope, dim3(groups, n, 1), dim3(256), (hipStream_t)stream, &a, sizeof a);
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }
// Workspace of the pre-widened prefill over kv_len keys: f16 K and V rows [n_kv][kv_len][hd], and for the int8
// cache f32 K and V scales [n_kv][kv_len], each region 256-byte aligned.
size_t prefill_ws_bytes(int kv_len, int n_kv, int hd, int fmt) {
    const size_t rows = align256((size_t)n_kv * kv_len * hd * 2), scales = fmt == 1 ? align256((size_t)n_kv * kv_len * 4) : 0;
    return 2 * rows + 2 * scales;
}

// gi_attn_prefill, gi_attn_prefill_i8 and gi_attn_prefill_q4: the same launch with the f16, int8 or 4-bit kernel
// (fmt 0, 1, 2). With a workspace (int8 and 4-bit caches, head sizes 64, 128, 256) the keys 0..pos0+n-1 are first
// widened into it (gi_kv_widen) and the prefill stages the widened tiles by LDS-DMA, as it stages the f16 cache.
int prefill_impl(void* stream, const void* q, int q_dtype, long long q_stride, const void* kc, const void* vc,
                 const float* ks, const float* vs, long long sc_stride, long long sc_head_stride, int fmt,
                 long long kv_stride, long long kv_head_stride, void* out, int out_dtype, long long out_stride, int pos0,
                 int n, int n_heads, int n_kv, int hd, float scale, void* workspace = nullptr,
                 size_t workspace_bytes = 0, bool f32_prompt = false) {
    const bool i8 = fmt == 1;
    if (int e = check_shape(n_heads, n_kv, hd, true)) return e;
    if (fmt == 2 && hd != 256) return fail("the 4-bit cache takes head size 256 only (got %d)", hd);
    if (f32_prompt && (fmt == 2 || hd > 128))
        return fail("f32 prompts take the f16 and int8 caches at head sizes up to 128 (the reference's attention_prefill)");
    if (n <= 0 || pos0 < 0) return fail("n %d must be positive and pos0 %d >= 0", n, pos0);
    if (!q || !kc || !vc || !out) return fail("null tensor pointer");
    if ((q_dtype != GI_F32 && q_dtype != GI_F16) || (out_dtype != GI_F32 && out_dtype != GI_F16))
        return fail("dtypes must be GI_F32 or GI_F16");
    if (fmt == 2) {
        // rows of 128 bytes (kv strides in bytes), 8 f16 scales a row (scale strides in f16 elements)
        if (kv_head_stride == 0) kv_head_stride = hd / 2;
        if (int e = check_kv_strides(kv_stride, kv_head_stride, n_kv, hd / 2, 16)) return e;
        if (!ks || !vs) return fail("null scale pointer");
        // (the kernels read a row's scales in 4-byte words)
        if (((uintptr_t)ks & 3) || ((uintptr_t)vs & 3) || ((sc_stride | sc_head_stride) & 1))
            return fail("ks and vs must be 4-byte aligned and their strides even");
        if (int e = check_kv_strides(sc_stride, sc_head_stride, n_kv, 8, 1)) return e;
    } else {
        if (kv_head_stride == 0) kv_head_stride = hd;
        if (int e = check_kv_strides(kv_stride, kv_head_stride, n_kv, hd, fmt ? 16 : 8)) return e;
        if (fmt)
            if (int e = check_scales(ks, vs, sc_stride, sc_head_stride)) return e;
    }
    if (!aligned16(q) || !aligned16(kc) || !aligned16(vc) || !aligned16(out) ||
        q_stride % (q_dtype == GI_F16 ? 8 : 4) || out_stride % (out_dtype == GI_F16 ? 8 : 4))
        return fail("tensors must be 16-byte aligned with row strides of whole 16-byte units");
    if (q_stride < (long long)n_heads * hd || out_stride < (long long)n_heads * hd)
        return fail("row strides too small for %d heads", n_heads);
    Module* m;
    if (int e = load_module(nullptr, &m)) return e;
    GiPrefillArgs a{};
    a.q = q;
    a.kc = (const uint16_t*)kc;
    a.vc = (const uint16_t*)vc;
    if (fmt) {
        a.ks = ks;
        a.vs = vs;
        a.sc_stride = sc_stride;
        a.sc_head_stride = sc_head_stride;
    }
    a.out = out;
    a.q_stride = q_stride;
    a.kv_stride = kv_stride;
    a.out_stride = out_stride;
    a.kv_head_stride = kv_head_stride;
    a.pos0 = pos0;
    a.n = n;
    a.n_heads = n_heads;
    a.n_kv = n_kv;
    a.qscale = scale * kLog2e;
    a.q_f16 = q_dtype == GI_F16;
    a.out_f16 = out_dtype == GI_F16;
    a.hd = hd;
    if (f32_prompt && !f32_hd(hd)) // head sizes 64 and 128 in f32: one workgroup per (head, 128 query rows)
        return launch(kPrefill, m->prefill_f32p[i8][hd == 128], dim3((n + kF32Rows - 1) / kF32Rows * n_heads, 1, 1),
                      dim3(kF32Threads), (hipStream_t)stream, &a, sizeof a);
    if (fmt && workspace && !f32_hd(hd)) {
        const int len = pos0 + n;
        const size_t need = prefill_ws_bytes(len, n_kv, hd, fmt);
        if (workspace_bytes < need)
            return fail("the prefill workspace holds %zu bytes; %zu needed (gi_attn_prefill_workspace_bytes)",
                        workspace_bytes, need);
        if ((uintptr_t)workspace & 255) return fail("the prefill workspace must be 256-byte aligned");
        unsigned char* w = (unsigned char*)workspace;
        const size_t rows = align256((size_t)n_kv * len * hd * 2), scales = fmt == 1 ? align256((size_t)n_kv * len * 4) : 0;
        GiWidenArgs wa{};
        wa.kc = kc;
        wa.vc = vc;
        wa.ks = ks;
        wa.vs = vs;
        wa.kw = w;
        wa.vw = w + rows;
        wa.ksw = fmt == 1 ? (float*)(w + 2 * rows) : nullptr;
        wa.vsw = fmt == 1 ? (float*)(w + 2 * rows + scales) : nullptr;
        wa.kv_stride = kv_stride;
        wa.kv_head_stride = kv_head_stride;
        wa.sc_stride = sc_stride;
        wa.sc_head_stride = sc_head_stride;
        wa.n_rows = len;
        wa.n_kv = n_kv;
        wa.hd = hd;
        wa.fmt = fmt;
        wa.vbias = hd == 256 ? 1.f : kPrefillI8VBias;
        const long long units = (long long)n_kv * len * (hd / 8);
        const unsigned blocks = (unsigned)std::min<long long>((units + 255) / 256, 8192);
        if (int e = launch(kWiden, m->widen, dim3(blocks), dim3(256), (hipStream_t)stream, &wa, sizeof wa)) return e;
        a.kc = (const uint16_t*)wa.kw;
        a.vc = (const uint16_t*)wa.vw;
        a.kv_stride = hd;
        a.kv_head_stride = (long long)len * hd;
        a.ks = wa.ksw;
        a.vs = wa.vsw;
        a.sc_stride = 1;
        a.sc_head_stride = len;
        if (hd == 256)
            return launch(kPrefill, fmt == 2 ? m->prefill256r : m->prefill_i8s[2],
                          dim3((n + kPrefill256rRows - 1) / kPrefill256rRows * n_heads, 1, 1), dim3(m->prefill256r_threads),
                          (hipStream_t)stream, &a, sizeof a);
        return launch(kPrefill, m->prefill_i8s[hd == 64 ? 1 : 0], dim3((n + kPrefillRows - 1) / kPrefillRows * n_heads, 1, 1),
                      dim3(m->prefill_threads[1]), (hipStream_t)stream, &a, sizeof a);
    }
    if (f32_hd(hd)) // one workgroup per (head, 128 query rows)
        return launch(kPrefill, m->prefill_f32[i8][f32_index(hd)], dim3((n + kF32Rows - 1) / kF32Rows * n_heads, 1, 1),
                      dim3(kF32Threads), (hipStream_t)stream, &a, sizeof a);
    if (hd == 256) // one workgroup per (head, 128 query rows), 16 rows per wave
        return launch(kPrefill, fmt ? m->prefill256r_fmt[fmt - 1] : m->prefill256r, dim3((n + kPrefill256rRows - 1) / kPrefill256rRows * n_heads, 1, 1),
                      dim3(m->prefill256r_threads), (hipStream_t)stream, &a, sizeof a);
    const int qtiles = (n + kPrefillRows - 1) / kPrefillRows; // one workgroup per (head, 256 query rows)
    return launch(kPrefill, hd == 64 ? m->prefill64[i8] : m->prefill[i8], dim3(qtiles * n_heads, 1, 1),
                  dim3(m->prefill_threads[i8]),
                  (hipStream_t)stream, &a, sizeof a);
}

int attention_impl(void* stream, const float* qkv, const void* kc, const void* vc, const float* ks, const float* vs,
                   int fmt, float* out, void* workspace, size_t workspace_bytes, int pos0, const int* posp, int ctx_cap,
                   int n, int n_heads, int n_kv, int hd, int exact);

} // namespace

extern "C" {

int gi_init(const char* code_object_path) {
    Module* m;
    return load_module(code_object_path, &m);
}

const char* gi_last_error(void) { return g_err.c_str(); }

int gi_attn_decode_plan(int max_span, int n_tok, int n_heads, int n_kv, int hd, int* chunk, int* nsplit) {
    if (int e = check_shape(n_heads, n_kv, hd, true)) return e;
    if (max_span <= 0 || n_tok <= 0) return fail("max_span %d and n_tok %d must be positive", max_span, n_tok);
    if (!chunk || !nsplit) return fail("null output pointer");
    plan(max_span, n_tok, n_heads, n_kv, chunk, nsplit, slice_unit(false, hd), hd);
    return 0;
}

size_t gi_attn_decode_workspace_bytes(int ctx_cap, int n_tok, int n_heads, int n_kv, int hd) {
    if (check_shape(n_heads, n_kv, hd, true) || ctx_cap <= 0 || n_tok <= 0) return 0;
    // the most partials any launch of up to n_tok tokens whose spans reach at most ctx_cap keys writes:
    // plan() caps the slices per (kv head, pair group) at per_slot, and a span never has more slices
    // than slice units (the smallest unit of the head size, f16's)
    const int unit = slice_unit(false, hd);
    size_t best = 16;
    int G = n_heads / n_kv;
    for (int t = 1; t <= n_tok; t++)
        for (int fmt = 0; fmt < (hd == 256 ? 3 : 2); fmt++) {
            int groups = dec_variant(t, G, hd, fmt).groups;
            int per_slot = slices_per_slot(n_heads, n_kv, groups, hd);
            int most = std::max(1, std::min(per_slot, (ctx_cap + unit - 1) / unit));
            best = std::max(best, (size_t)t * n_heads * most * (hd + 4) * sizeof(float));
        }
    return best;
}

int gi_attn_decode(void* stream, const float* q, long long q_stride, const uint16_t* kc, const uint16_t* vc,
                   long long kv_stride, long long kv_head_stride, float* out, long long out_stride, void* workspace,
                   size_t workspace_bytes, int pos0, const int* posp, int ctx_cap, int n_tok, int n_heads, int n_kv,
                   int hd, float scale) {
    return decode_impl(stream, q, q_stride, kc, vc, nullptr, nullptr, 0, 0, false, kv_stride, kv_head_stride, out,
                       out_stride, workspace, workspace_bytes, pos0, posp, ctx_cap, n_tok, n_heads, n_kv, hd, scale);
}

int gi_attn_decode_noalloc(void* stream, const float* q, long long q_stride, const uint16_t* kc, const uint16_t* vc,
                           long long kv_stride, long long kv_head_stride, float* out, long long out_stride, int pos0,
                           const int* posp, int ctx_cap, int n_tok, int n_heads, int n_kv, int hd, float scale) {
    if (int e = check_shape(n_heads, n_kv, hd, true)) return e;
    if (n_tok <= 0) return fail("n_tok %d must be positive", n_tok);
    Module* m;
    if (int e = load_module(nullptr, &m)) return e;
    // the partials this call needs (decode_impl repeats the plan and every other check)
    int chunk = 0, nsplit = 0;
    plan(posp ? std::max(ctx_cap, 1) : std::max(pos0 + n_tok, 1), n_tok, n_heads, n_kv, &chunk, &nsplit,
         slice_unit(false, hd), hd);
    const size_t need = nsplit == 1 ? 0 : (size_t)n_tok * n_heads * nsplit * (hd + 4) * sizeof(float);
    if (need > m->scratch_bytes)
        return fail("gi_attn_decode_noalloc: %zu bytes of slice partials exceed the %zu-byte scratch (use "
                    "gi_attn_decode with a workspace)", need, m->scratch_bytes);
    return decode_impl(stream, q, q_stride, kc, vc, nullptr, nullptr, 0, 0, false, kv_stride, kv_head_stride, out,
                       out_stride, m->scratch, m->scratch_bytes, pos0, posp, ctx_cap, n_tok, n_heads, n_kv, hd, scale);
}

int gi_attn_decode_i8(void* stream, const float* q, long long q_stride, const int8_t* kc, const int8_t* vc,
                      const float* ks, const float* vs, long long kv_stride, long long kv_head_stride,
                      long long sc_stride, long long sc_head_stride, float* out, long long out_stride, void* workspace,
                      size_t workspace_bytes, int pos0, const int* posp, int ctx_cap, int n_tok, int n_heads, int n_kv,
                      int hd, float scale) {
    if (sc_stride == 0 && sc_head_stride == 0) sc_stride = n_kv, sc_head_stride = 1;
    return decode_impl(stream, q, q_stride, kc, vc, ks, vs, sc_stride, sc_head_stride, true, kv_stride, kv_head_stride,
                       out, out_stride, workspace, workspace_bytes, pos0, posp, ctx_cap, n_tok, n_heads, n_kv, hd, scale);
}

int gi_attn_decode_q4(void* stream, const float* q, long long q_stride, const uint8_t* kc, const uint8_t* vc,
                      const uint16_t* ks, const uint16_t* vs, long long kv_stride, long long kv_head_stride,
                      long long sc_stride, long long sc_head_stride, float* out, long long out_stride, void* workspace,
                      size_t workspace_bytes, int pos0, const int* posp, int ctx_cap, int n_tok, int n_heads, int n_kv,
                      float scale) {
    if (sc_stride == 0 && sc_head_stride == 0) sc_stride = 8LL * n_kv, sc_head_stride = 8;
    return decode_impl(stream, q, q_stride, kc, vc, (const float*)ks, (const float*)vs, sc_stride, sc_head_stride, 2,
                       kv_stride, kv_head_stride, out, out_stride, workspace, workspace_bytes, pos0, posp, ctx_cap, n_tok,
                       n_heads, n_kv, 256, scale);
}

int gi_attn_prefill(void* stream, const void* q, int q_dtype, long long q_stride, const uint16_t* kc,
                    const uint16_t* vc, long long kv_stride, long long kv_head_stride, void* out, int out_dtype,
                    long long out_stride, int pos0, int n, int n_heads, int n_kv, int hd, float scale) {
    return prefill_impl(stream, q, q_dtype, q_stride, kc, vc, nullptr, nullptr, 0, 0, false, kv_stride, kv_head_stride,
                        out, out_dtype, out_stride, pos0, n, n_heads, n_kv, hd, scale);
}

int gi_attn_prefill_i8(void* stream, const void* q, int q_dtype, long long q_stride, const int8_t* kc, const int8_t* vc,
                       const float* ks, const float* vs, long long kv_stride, long long kv_head_stride,
                       long long sc_stride, long long sc_head_stride, void* out, int out_dtype, long long out_stride,
                       int pos0, int n, int n_heads, int n_kv, int hd, float scale) {
    if (sc_stride == 0 && sc_head_stride == 0) sc_stride = n_kv, sc_head_stride = 1;
    return prefill_impl(stream, q, q_dtype, q_stride, kc, vc, ks, vs, sc_stride, sc_head_stride, true, kv_stride,
                        kv_head_stride, out, out_dtype, out_stride, pos0, n, n_heads, n_kv, hd, scale);
}

int gi_attn_prefill_q4(void* stream, const void* q, int q_dtype, long long q_stride, const uint8_t* kc,
                       const uint8_t* vc, const uint16_t* ks, const uint16_t* vs, long long kv_stride,
                       long long kv_head_stride, long long sc_stride, long long sc_head_stride, void* out, int out_dtype,
                       long long out_stride, int pos0, int n, int n_heads, int n_kv, float scale) {
    if (sc_stride == 0 && sc_head_stride == 0) sc_stride = 8LL * n_kv, sc_head_stride = 8;
    return prefill_impl(stream, q, q_dtype, q_stride, kc, vc, (const float*)ks, (const float*)vs, sc_stride,
                        sc_head_stride, 2, kv_stride, kv_head_stride, out, out_dtype, out_stride, pos0, n, n_heads, n_kv,
                        256, scale);
}

int gi_attn_prefill_f32(void* stream, const void* q, int q_dtype, long long q_stride, const void* kc, const void* vc,
                        const float* ks, const float* vs, int kv_int8, long long kv_stride, long long kv_head_stride,
                        long long sc_stride, long long sc_head_stride, void* out, int out_dtype, long long out_stride,
                        int pos0, int n, int n_heads, int n_kv, int hd, float scale) {
    if (kv_int8 && sc_stride == 0 && sc_head_stride == 0) sc_stride = n_kv, sc_head_stride = 1;
    return prefill_impl(stream, q, q_dtype, q_stride, kc, vc, kv_int8 ? ks : nullptr, kv_int8 ? vs : nullptr,
                        kv_int8 ? sc_stride : 0, kv_int8 ? sc_head_stride : 0, kv_int8 ? 1 : 0, kv_stride,
                        kv_head_stride, out, out_dtype, out_stride, pos0, n, n_heads, n_kv, hd, scale, nullptr, 0, true);
}

size_t gi_attn_prefill_workspace_bytes(int kv_len, int n_kv, int hd, int fmt) {
    if (kv_len <= 0 || n_kv <= 0 || (fmt != 1 && fmt != 2) || (hd != 64 && hd != 128 && hd != 256) ||
        (fmt == 2 && hd != 256))
        return 0;
    return prefill_ws_bytes(kv_len, n_kv, hd, fmt);
}

int gi_attn_prefill_i8_ws(void* stream, const void* q, int q_dtype, long long q_stride, const int8_t* kc,
                          const int8_t* vc, const float* ks, const float* vs, long long kv_stride,
                          long long kv_head_stride, long long sc_stride, long long sc_head_stride, void* out,
                          int out_dtype, long long out_stride, int pos0, int n, int n_heads, int n_kv, int hd,
                          float scale, void* workspace, size_t workspace_bytes) {
    if (!workspace) return fail("null workspace");
    if (sc_stride == 0 && sc_head_stride == 0) sc_stride = n_kv, sc_head_stride = 1;
    return prefill_impl(stream, q, q_dtype, q_stride, kc, vc, ks, vs, sc_stride, sc_head_stride, 1, kv_stride,
                        kv_head_stride, out, out_dtype, out_stride, pos0, n, n_heads, n_kv, hd, scale, workspace,
                        workspace_bytes);
}

int gi_attn_prefill_q4_ws(void* stream, const void* q, int q_dtype, long long q_stride, const uint8_t* kc,
                          const uint8_t* vc, const uint16_t* ks, const uint16_t* vs, long long kv_stride,
                          long long kv_head_stride, long long sc_stride, long long sc_head_stride, void* out,
                          int out_dtype, long long out_stride, int pos0, int n, int n_heads, int n_kv, float scale,
                          void* workspace, size_t workspace_bytes) {
    if (!workspace) return fail("null workspace");
    if (sc_stride == 0 && sc_head_stride == 0) sc_stride = 8LL * n_kv, sc_head_stride = 8;
    return prefill_impl(stream, q, q_dtype, q_stride, kc, vc, (const float*)ks, (const float*)vs, sc_stride,
                        sc_head_stride, 2, kv_stride, kv_head_stride, out, out_dtype, out_stride, pos0, n, n_heads, n_kv,
                        256, scale, workspace, workspace_bytes);
}

int gi_attention(void* stream, const float* qkv, const uint16_t* kc, const uint16_t* vc, float* out,
                 void* workspace, size_t workspace_bytes, int pos0, const int* posp, int ctx_cap, int n, int n_heads,
                 int n_kv, int hd, int exact) {
    return attention_impl(stream, qkv, kc, vc, nullptr, nullptr, 0, out, workspace, workspace_bytes, pos0, posp,
                          ctx_cap, n, n_heads, n_kv, hd, exact);
}

int gi_attention_i8(void* stream, const float* qkv, const int8_t* kc, const int8_t* vc, const float* ks,
                    const float* vs, float* out, void* workspace, size_t workspace_bytes, int pos0, const int* posp,
                    int ctx_cap, int n, int n_heads, int n_kv, int hd, int exact) {
    return attention_impl(stream, qkv, kc, vc, ks, vs, 1, out, workspace, workspace_bytes, pos0, posp, ctx_cap, n,
                          n_heads, n_kv, hd, exact);
}

int gi_attention_q4(void* stream, const float* qkv, const uint8_t* kc, const uint8_t* vc, const uint16_t* ks,
                    const uint16_t* vs, float* out, void* workspace, size_t workspace_bytes, int pos0, const int* posp,
                    int ctx_cap, int n, int n_heads, int n_kv, int exact) {
    return attention_impl(stream, qkv, kc, vc, (const float*)ks, (const float*)vs, 2, out, workspace, workspace_bytes,
                          pos0, posp, ctx_cap, n, n_heads, n_kv, 256, exact);
}

int gi_hadamard_rows(void* stream, float* x, long long row_stride, int rows, int width) {
    if (rows < 0 || width <= 0 || width % 256) return fail("rows %d >= 0 and width %d (a multiple of 256) required", rows, width);
    if (rows == 0) return 0;
    if (!x) return fail("null tensor pointer");
    if (!aligned16(x) || row_stride % 4 || row_stride < width)
        return fail("x must be 16-byte aligned with a row stride (a multiple of 4, >= width)");
    Module* m;
    if (int e = load_module(nullptr, &m)) return e;
    GiHadamardArgs a{x, row_stride, rows, width / 256};
    const long long segs = (long long)rows * a.segs;
    return launch(kHadamard, m->hadamard, dim3((unsigned)((segs + 3) / 4)), dim3(256), (hipStream_t)stream, &a,
                  sizeof a);
}

} // extern "C"

namespace {
// GpuModel::attention's dispatch over either cache type (the reference's layout, scales [pos][n_kv]).
int attention_impl(void* stream, const float* qkv, const void* kc, const void* vc, const float* ks, const float* vs,
                   int fmt, float* out, void* workspace, size_t workspace_bytes, int pos0, const int* posp, int ctx_cap,
                   int n, int n_heads, int n_kv, int hd, int exact) {
    if (int e = check_shape(n_heads, n_kv, hd, true)) return e;
    if (n <= 0) return fail("n %d must be positive", n);
    const long long q_dim = (long long)n_heads * hd, kv_dim = (long long)n_kv * hd, row = q_dim + 2 * kv_dim;
    const float scale = 1.0f / std::sqrt((float)hd);
    // the reference's cache layouts: [position][n_kv][hd] rows (the 4-bit cache: hd / 2 bytes a row) and scales
    // [position][n_kv] (the 4-bit cache: [position][n_kv][hd / 32] f16)
    const long long kvs = fmt == 2 ? kv_dim / 2 : kv_dim, kvh = fmt == 2 ? hd / 2 : hd;
    const long long scs = fmt == 2 ? (long long)n_kv * (hd / 32) : n_kv, sch = fmt == 2 ? hd / 32 : 1;
    // exact bit 0: a verify batch, every token on the split path (s.exact, src/cuda.rs:8457-8458). Bit 1: the
    // reference with its tensor-core kernels off (GHOST_INFER_NO_TC_ATT): prompts in f32 (attention_prefill, head sizes
    // up to 128, src/cuda.rs:8452-8476; the 4-bit cache and head size 256 have no such kernel there and take the split
    // path), and the head-256 int8 decode in f32 precision (no attention_decode_tc256, src/cuda.rs:5655)
    const bool verify = exact & 1, no_tc = exact & 2;
    if (n >= kTiledMinBatch && !verify && no_tc && fmt != 2 && hd <= 128) {
        if (posp) return fail("a device position (posp) is only taken by the split path");
        return prefill_impl(stream, qkv, GI_F32, row, kc, vc, ks, vs, scs, sch, fmt, kvs, kvh, out, GI_F32, q_dim, pos0,
                            n, n_heads, n_kv, hd, scale, nullptr, 0, true);
    }
    if (n >= kTiledMinBatch && !verify && !no_tc) {
        if (posp) return fail("a device position (posp) is only taken by the split path");
        // the int8 and 4-bit caches: pre-widened staging when the workspace holds it
        const bool staged = fmt && workspace && workspace_bytes >= prefill_ws_bytes(pos0 + n, n_kv, hd, fmt);
        return prefill_impl(stream, qkv, GI_F32, row, kc, vc, ks, vs, scs, sch, fmt, kvs, kvh, out, GI_F32, q_dim, pos0,
                            n, n_heads, n_kv, hd, scale, staged ? workspace : nullptr, workspace_bytes);
    }
    for (int b0 = 0; b0 < n; b0 += kSplitMaxBatch) {
        int m = std::min(n - b0, kSplitMaxBatch);
        // with a device position every launch reads *posp, so only single launches take it
        if (posp && n > kSplitMaxBatch) return fail("posp takes at most %d tokens", kSplitMaxBatch);
        if (int e = decode_impl(stream, qkv + b0 * row, row, kc, vc, ks, vs, scs, sch, fmt, kvs, kvh, out + b0 * q_dim,
                                q_dim, workspace, workspace_bytes, pos0 + b0, posp, ctx_cap, m, n_heads, n_kv, hd, scale,
                                no_tc))
            return e;
    }
    return 0;
}
} // namespace

extern "C" {


int gi_kernel_timing(int on) {
    std::lock_guard<std::mutex> lock(g_timing.mu);
    g_timing.on = on != 0;
    return 0;
}

int gi_kernel_timing_read(const char* kernel, double* total_ms, int* launches) {
    if (!kernel || !total_ms || !launches) return fail("gi_kernel_timing_read: null argument");
    int kind = -1;
    for (int k = 0; k < kKinds; k++)
        if (std::strcmp(kernel, kKindNames[k]) == 0) kind = k;
    if (kind < 0)
        return fail("unknown kernel \"%s\" (decode_partial, decode_combine, prefill, qk_norm_rope, kv_relayout, "
                    "hadamard_rows or kv_widen)", kernel);
    std::vector<std::pair<hipEvent_t, hipEvent_t>> ev;
    {
        std::lock_guard<std::mutex> lock(g_timing.mu);
        ev.swap(g_timing.ev[kind]);
    }
    double sum = 0.0;
    int err = 0;
    for (auto& p : ev) {
        float ms = 0.f;
        if (!err) err = check(hipEventSynchronize(p.second), "hipEventSynchronize");
        if (!err) err = check(hipEventElapsedTime(&ms, p.first, p.second), "hipEventElapsedTime");
        sum += ms;
        (void)hipEventDestroy(p.first);
        (void)hipEventDestroy(p.second);
    }
    *total_ms = sum;
    *launches = (int)ev.size();
    return err;
}

int gi_qk_norm_rope(void* stream, float* qkv, const float* qn, const float* kn, uint16_t* kc, uint16_t* vc,
                    long long kv_stride, long long kv_head_stride, int pos0, const int* posp, int ctx_cap, int n,
                    int n_heads, int n_kv, int hd, int rope_dim, float base, const float* ff, int neox, float eps) {
    return rope_impl(stream, qkv, qn, kn, kc, vc, nullptr, nullptr, 0, 0, 0, kv_stride, kv_head_stride, pos0, posp,
                     ctx_cap, n, n_heads, n_kv, hd, rope_dim, base, ff, neox, eps);
}

int gi_qk_norm_rope_i8(void* stream, float* qkv, const float* qn, const float* kn, int8_t* kc, int8_t* vc, float* ks,
                       float* vs, long long kv_stride, long long kv_head_stride, long long sc_stride,
                       long long sc_head_stride, int pos0, const int* posp, int ctx_cap, int n, int n_heads, int n_kv,
                       int hd, int rope_dim, float base, const float* ff, int neox, float eps) {
    if (sc_stride == 0 && sc_head_stride == 0) sc_stride = n_kv, sc_head_stride = 1;
    return rope_impl(stream, qkv, qn, kn, kc, vc, ks, vs, sc_stride, sc_head_stride, 1, kv_stride, kv_head_stride,
                     pos0, posp, ctx_cap, n, n_heads, n_kv, hd, rope_dim, base, ff, neox, eps);
}

int gi_qk_norm_rope_q4(void* stream, float* qkv, const float* qn, const float* kn, uint8_t* kc, uint8_t* vc,
                       uint16_t* ks, uint16_t* vs, long long kv_stride, long long kv_head_stride, long long sc_stride,
                       long long sc_head_stride, int pos0, const int* posp, int ctx_cap, int n, int n_heads, int n_kv,
                       int rope_dim, float base, const float* ff, int neox, float eps) {
    if (sc_stride == 0 && sc_head_stride == 0) sc_stride = 8LL * n_kv, sc_head_stride = 8;
    return rope_impl(stream, qkv, qn, kn, kc, vc, (float*)ks, (float*)vs, sc_stride, sc_head_stride, 2, kv_stride,
                     kv_head_stride, pos0, posp, ctx_cap, n, n_heads, n_kv, 256, rope_dim, base, ff, neox, eps);
}

int gi_kv_relayout(void* stream, const void* src, long long src_stride, long long src_head_stride, void* dst,
                   long long dst_stride, long long dst_head_stride, int n_rows, int n_kv, int row_bytes) {
    if (n_rows < 0 || n_kv <= 0 || row_bytes <= 0 || row_bytes % 4)
        return fail("n_rows %d >= 0, n_kv %d > 0 and row_bytes %d (a positive multiple of 4) required", n_rows, n_kv,
                    row_bytes);
    if (n_rows == 0) return 0;
    if (!src || !dst) return fail("null tensor pointer");
    if (((uintptr_t)src | (uintptr_t)dst) & 3 || (src_stride | src_head_stride | dst_stride | dst_head_stride) & 3)
        return fail("pointers and strides must be multiples of 4 bytes");
    if (src_stride <= 0 || src_head_stride <= 0 || dst_stride <= 0 || dst_head_stride <= 0)
        return fail("strides must be positive");
    // the two sides' spans must not overlap (rows would be read after they are overwritten)
    auto span = [&](const void* p, long long st, long long hs) {
        const uintptr_t b = (uintptr_t)p;
        return std::make_pair(b, b + (uintptr_t)((long long)(n_rows - 1) * st + (long long)(n_kv - 1) * hs + row_bytes));
    };
    const auto s = span(src, src_stride, src_head_stride), d = span(dst, dst_stride, dst_head_stride);
    if (s.first < d.second && d.first < s.second) return fail("source and destination overlap");
    Module* m;
    if (int e = load_module(nullptr, &m)) return e;
    GiRelayoutArgs a{};
    const bool wide = !(((uintptr_t)src | (uintptr_t)dst) & 15) && !((src_stride | src_head_stride | dst_stride |
                                                                      dst_head_stride | row_bytes) & 15);
    a.src = src;
    a.dst = dst;
    a.src_stride = src_stride;
    a.src_head_stride = src_head_stride;
    a.dst_stride = dst_stride;
    a.dst_head_stride = dst_head_stride;
    a.n_rows = n_rows;
    a.unit = wide ? 16 : 4;
    a.units_per_row = row_bytes / a.unit;
    a.n_units = (long long)n_kv * n_rows * a.units_per_row;
    const long long wgs = std::min<long long>((a.n_units + 255) / 256, 256 * 16);
    return launch(kRelayout, m->relayout, dim3((unsigned)wgs), dim3(256), (hipStream_t)stream, &a, sizeof a);
}

} // extern "C"
