// gi_layer_harness: the caller side of the attention operator, driven the way the reference's layer loop
// drives it (layer_attn, src/cuda.rs:9706-9717: qk_norm_rope with the cache store, then
// GpuModel::attention, src/cuda.rs:8448-8541), for one layer, through the C ABI of include/gi_attn.h:
//   1. a prompt of --prompt tokens: one cache write and one attention call (the prefill path for >= 16
//      tokens);
//   2. --steps decode steps, one token each: the cache write and the split path at the next position. With
//      --graph (the default) the step is captured once into a HIP graph and replayed with the position in
//      device memory, the session's fixed row buffers standing in for the engine's (src/cuda.rs:8686-8712);
//   3. a reference pass: attention over the whole sequence on the exact split path (verify blocks of up to
//      15 tokens), with every output row checked against it: prompt rows within the path's parity bar
//      (max-abs 2e-3: the prefill rounds P to f16), decoded rows within 2e-5 (both sides compute in f32
//      precision; 1e-3 at head size 256 over the int8 and 4-bit caches, whose split path rounds Q and P to f16
//      as the reference's attention_decode_tc256 does).
// --q4 (head size 256) plays the reference's 4-bit cache: the cache write rotates q, k and v rows, and every
// attention call is followed by gi_hadamard_rows on its output rows, as the layer does (src/cuda.rs:9765-9768).
// One JSON line goes to stdout. Exit status 0 when every row agrees, 1 when one does not, 2 on a usage or
// runtime error. The harness owns all memory (hipMalloc); the library it calls allocates nothing.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "gi_attn.h"

namespace {

struct Opts {
    int prompt = 300, steps = 24, heads = 32, kv = 8, hd = 128, seed = 1;
    bool i8 = false, q4 = false, graph = true;
    std::string dump; // file for the final qkv rows and the output rows (f32, raw), for checks outside
};

[[noreturn]] void die(const std::string& what) {
    fprintf(stderr, "gi_layer_harness: %s\n", what.c_str());
    exit(2);
}
void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) die(std::string(what) + ": " + hipGetErrorString(e));
}
void gi_ok(int rc, const char* what) {
    if (rc != 0) die(std::string(what) + ": " + gi_last_error());
}

void usage() {
    printf("usage: gi_layer_harness [--prompt N] [--steps S] [--heads H] [--kv K] [--hd 64|128|256|16..112] [--int8 | --q4]\n"
           "                        [--no-graph] [--seed X] [--dump FILE]\n"
           "Plays one layer's attention through the C ABI (cache write + prefill for the prompt, then one\n"
           "decode step per token, replayed from a HIP graph), checks every output row against the exact\n"
           "split path over the whole sequence, and prints one JSON line. --dump writes the rotated qkv rows\n"
           "and the output rows (f32) to FILE.\n");
}

Opts parse(int argc, char** argv) {
    Opts o;
    for (int i = 1; i < argc; i++) {
        std::string a = argv[i];
        auto num = [&](int& v) {
            if (i + 1 >= argc) die("missing value after " + a);
            v = atoi(argv[++i]);
        };
        if (a == "--help" || a == "-h") {
            usage();
            exit(0);
        } else if (a == "--prompt") num(o.prompt);
        else if (a == "--steps") num(o.steps);
        else if (a == "--heads") num(o.heads);
        else if (a == "--kv") num(o.kv);
        else if (a == "--hd") num(o.hd);
        else if (a == "--seed") num(o.seed);
        else if (a == "--int8") o.i8 = true;
        else if (a == "--q4") o.q4 = true;
        else if (a == "--no-graph") o.graph = false;
        else if (a == "--dump") {
            if (i + 1 >= argc) die("missing value after --dump");
            o.dump = argv[++i];
        }
        else die("unknown argument " + a);
    }
    const bool f32_hd = o.hd % 16 == 0 && o.hd >= 16 && o.hd <= 112 && o.hd != 64; // the f32 kernels' sizes
    if (o.prompt < 1 || o.steps < 0 || o.heads < 1 || o.kv < 1 || o.heads % o.kv ||
        (o.hd != 64 && o.hd != 128 && o.hd != 256 && !f32_hd) || (o.q4 && (o.hd != 256 || o.i8)))
        die("bad shape (heads a multiple of kv; hd 64, 128, 256 or a multiple of 16 up to 112; --q4 takes hd 256 "
            "and not --int8)");
    return o;
}

template <typename T> T* dev_alloc(size_t n) {
    void* p = nullptr;
    hip_ok(hipMalloc(&p, n * sizeof(T) + 16), "hipMalloc");
    return static_cast<T*>(p);
}

} // namespace

int main(int argc, char** argv) {
    const Opts o = parse(argc, argv);
    const int H = o.heads, K = o.kv, hd = o.hd, total = o.prompt + o.steps;
    const int cap = (total + 255) / 256 * 256;     // session capacity
    const long long row = (long long)(H + 2 * K) * hd; // qkv row: [q | k | v]
    const long long orow = (long long)H * hd;
    const int rope_dim = hd;
    const float rope_base = 1e6f, eps = 1e-6f;

    hip_ok(hipSetDevice(0), "hipSetDevice");
    hipStream_t st;
    hip_ok(hipStreamCreate(&st), "hipStreamCreate");
    gi_ok(gi_init(nullptr), "gi_init");

    // session buffers: qkv rows, outputs, head-major caches [kv][cap][hd] (and scales [kv][cap]), workspace
    std::vector<float> qkv_h((size_t)total * row);
    std::mt19937 gen(o.seed);
    std::normal_distribution<float> nd(0.f, 1.f);
    for (auto& x : qkv_h) x = nd(gen);
    float* qkv = dev_alloc<float>(qkv_h.size());
    float* out = dev_alloc<float>((size_t)total * orow);
    float* ref = dev_alloc<float>((size_t)total * orow);
    hip_ok(hipMemcpy(qkv, qkv_h.data(), qkv_h.size() * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy qkv");
    // head-major caches; the 4-bit one: rows of hd/2 bytes, hd/32 f16 scales a row
    const size_t cache_bytes = (size_t)K * cap * (o.q4 ? hd / 2 : o.i8 ? hd : 2 * hd);
    void* kc = dev_alloc<char>(cache_bytes);
    void* vc = dev_alloc<char>(cache_bytes);
    const size_t sc_bytes = (size_t)K * cap * (o.q4 ? hd / 16 : 4);
    float* ks = o.i8 || o.q4 ? (float*)dev_alloc<char>(sc_bytes) : nullptr;
    float* vs = o.i8 || o.q4 ? (float*)dev_alloc<char>(sc_bytes) : nullptr;
    const long long kv_stride = o.q4 ? hd / 2 : hd, kv_head_stride = (long long)cap * kv_stride;
    const long long sc_stride = o.q4 ? hd / 32 : 1, sc_head_stride = (long long)cap * sc_stride;
    // one workspace for the decode partials and, over the int8 and 4-bit caches, the prompt's widened keys
    const size_t part_bytes = gi_attn_decode_workspace_bytes(cap, 15, H, K, hd);
    if (part_bytes == 0) die("gi_attn_decode_workspace_bytes rejected the shape");
    const size_t widen_bytes = o.i8 || o.q4 ? gi_attn_prefill_workspace_bytes(cap, K, hd, o.q4 ? 2 : 1) : 0;
    const size_t ws_bytes = part_bytes > widen_bytes ? part_bytes : widen_bytes;
    void* ws = dev_alloc<char>(ws_bytes);
    // the engine's fixed per-step buffers: the current token's qkv row and output row, and its position
    float* cur_row = dev_alloc<float>(row);
    float* cur_out = dev_alloc<float>(orow);
    int* posp = dev_alloc<int>(1);
    int* pos_host = nullptr;
    hip_ok(hipHostMalloc((void**)&pos_host, sizeof(int), hipHostMallocDefault), "hipHostMalloc");

    auto write_cache = [&](float* rows, int pos0, const int* pp, int n) {
        if (o.q4)
            return gi_qk_norm_rope_q4(st, rows, nullptr, nullptr, (uint8_t*)kc, (uint8_t*)vc, (uint16_t*)ks,
                                      (uint16_t*)vs, kv_stride, kv_head_stride, sc_stride, sc_head_stride, pos0, pp,
                                      cap, n, H, K, rope_dim, rope_base, nullptr, 1, eps);
        if (o.i8)
            return gi_qk_norm_rope_i8(st, rows, nullptr, nullptr, (int8_t*)kc, (int8_t*)vc, ks, vs, kv_stride,
                                      kv_head_stride, sc_stride, sc_head_stride, pos0, pp, cap, n, H, K, hd, rope_dim,
                                      rope_base, nullptr, 1, eps);
        return gi_qk_norm_rope(st, rows, nullptr, nullptr, (uint16_t*)kc, (uint16_t*)vc, kv_stride, kv_head_stride,
                               pos0, pp, cap, n, H, K, hd, rope_dim, rope_base, nullptr, 1, eps);
    };
    // gi_attention takes the reference's [position][n_kv][hd] cache; the head-major session cache goes
    // through the decode / prefill entry points with its strides, as the operator would dispatch them
    auto attention_rotated = [&](const float* rows, float* o_rows, int pos0, const int* pp, int n, int exact) {
        const float scale = 1.f / sqrtf((float)hd);
        if (n >= 16 && !exact) {
            if (o.q4)
                return gi_attn_prefill_q4_ws(st, rows, GI_F32, row, (const uint8_t*)kc, (const uint8_t*)vc,
                                             (const uint16_t*)ks, (const uint16_t*)vs, kv_stride, kv_head_stride,
                                             sc_stride, sc_head_stride, o_rows, GI_F32, orow, pos0, n, H, K, scale, ws,
                                             ws_bytes);
            if (o.i8 && widen_bytes) // (the f32 kernels' head sizes take no widened keys)
                return gi_attn_prefill_i8_ws(st, rows, GI_F32, row, (const int8_t*)kc, (const int8_t*)vc, ks, vs,
                                             kv_stride, kv_head_stride, sc_stride, sc_head_stride, o_rows, GI_F32,
                                             orow, pos0, n, H, K, hd, scale, ws, ws_bytes);
            if (o.i8)
                return gi_attn_prefill_i8(st, rows, GI_F32, row, (const int8_t*)kc, (const int8_t*)vc, ks, vs,
                                          kv_stride, kv_head_stride, sc_stride, sc_head_stride, o_rows, GI_F32, orow,
                                          pos0, n, H, K, hd, scale);
            return gi_attn_prefill(st, rows, GI_F32, row, (const uint16_t*)kc, (const uint16_t*)vc, kv_stride,
                                   kv_head_stride, o_rows, GI_F32, orow, pos0, n, H, K, hd, scale);
        }
        for (int b0 = 0; b0 < n; b0 += 15) { // SPLIT_MAX_BATCH (src/cuda.rs:119)
            const int m = n - b0 < 15 ? n - b0 : 15;
            int rc = o.q4 ? gi_attn_decode_q4(st, rows + b0 * row, row, (const uint8_t*)kc, (const uint8_t*)vc,
                                              (const uint16_t*)ks, (const uint16_t*)vs, kv_stride, kv_head_stride,
                                              sc_stride, sc_head_stride, o_rows + b0 * orow, orow, ws, ws_bytes,
                                              pos0 + b0, pp, pp ? cap : 0, m, H, K, scale)
                   : o.i8 ? gi_attn_decode_i8(st, rows + b0 * row, row, (const int8_t*)kc, (const int8_t*)vc, ks, vs,
                                              kv_stride, kv_head_stride, sc_stride, sc_head_stride, o_rows + b0 * orow,
                                              orow, ws, ws_bytes, pos0 + b0, pp, pp ? cap : 0, m, H, K, hd, scale)
                          : gi_attn_decode(st, rows + b0 * row, row, (const uint16_t*)kc, (const uint16_t*)vc,
                                           kv_stride, kv_head_stride, o_rows + b0 * orow, orow, ws, ws_bytes,
                                           pos0 + b0, pp, pp ? cap : 0, m, H, K, hd, scale);
            if (rc) return rc;
        }
        return 0;
    };
    // the layer's attention step: a 4-bit cache's output rows are rotated back
    auto attention = [&](const float* rows, float* o_rows, int pos0, const int* pp, int n, int exact) {
        int rc = attention_rotated(rows, o_rows, pos0, pp, n, exact);
        if (!rc && o.q4) rc = gi_hadamard_rows(st, o_rows, orow, n, (int)orow);
        return rc;
    };

    hipEvent_t e0, e1;
    hip_ok(hipEventCreate(&e0), "hipEventCreate");
    hip_ok(hipEventCreate(&e1), "hipEventCreate");

    // progress on stderr, flushed, so that a run that stalls shows how far it got
    auto stage = [](const char* what) {
        fprintf(stderr, "[harness] %s\n", what);
        fflush(stderr);
    };
    // 1. the prompt
    stage("prompt");
    hip_ok(hipEventRecord(e0, st), "hipEventRecord");
    gi_ok(write_cache(qkv, 0, nullptr, o.prompt), "cache write (prompt)");
    gi_ok(attention(qkv, out, 0, nullptr, o.prompt, 0), "attention (prompt)");
    hip_ok(hipEventRecord(e1, st), "hipEventRecord");
    hip_ok(hipStreamSynchronize(st), "hipStreamSynchronize");
    float prompt_ms = 0.f;
    hip_ok(hipEventElapsedTime(&prompt_ms, e0, e1), "hipEventElapsedTime");

    // 2. decode steps
    stage("decode steps");
    hipGraphExec_t exec = nullptr;
    if (o.graph && o.steps > 0) {
        hipGraph_t graph;
        hip_ok(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        int rc = write_cache(cur_row, 0, posp, 1);
        if (!rc) rc = attention(cur_row, cur_out, 0, posp, 1, 1);
        hip_ok(hipStreamEndCapture(st, &graph), "hipStreamEndCapture");
        gi_ok(rc, "decode step (capture)");
        hip_ok(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
        hip_ok(hipGraphDestroy(graph), "hipGraphDestroy");
    }
    float step_ms = 0.f;
    for (int s = 0; s < o.steps; s++) {
        const int t = o.prompt + s;
        float* trow = qkv + (size_t)t * row;
        float* tout = out + (size_t)t * orow;
        hip_ok(hipEventRecord(e0, st), "hipEventRecord");
        if (exec) {
            *pos_host = t;
            hip_ok(hipMemcpyAsync(posp, pos_host, sizeof(int), hipMemcpyHostToDevice, st), "position");
            hip_ok(hipMemcpyAsync(cur_row, trow, row * sizeof(float), hipMemcpyDeviceToDevice, st), "row in");
            hip_ok(hipGraphLaunch(exec, st), "hipGraphLaunch");
            hip_ok(hipMemcpyAsync(trow, cur_row, row * sizeof(float), hipMemcpyDeviceToDevice, st), "row out");
            hip_ok(hipMemcpyAsync(tout, cur_out, orow * sizeof(float), hipMemcpyDeviceToDevice, st), "output");
        } else {
            gi_ok(write_cache(trow, t, nullptr, 1), "cache write (step)");
            gi_ok(attention(trow, tout, t, nullptr, 1, 1), "attention (step)");
        }
        hip_ok(hipEventRecord(e1, st), "hipEventRecord");
        hip_ok(hipStreamSynchronize(st), "hipStreamSynchronize"); // the engine samples the token here
        float ms = 0.f;
        hip_ok(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
        step_ms += ms;
    }

    // 3. the reference pass over the whole (already rotated) sequence, exact split path
    stage("reference pass");
    gi_ok(attention(qkv, ref, 0, nullptr, total, 1), "attention (reference pass)");
    hip_ok(hipStreamSynchronize(st), "hipStreamSynchronize");
    std::vector<float> got((size_t)total * orow), want((size_t)total * orow);
    hip_ok(hipMemcpy(got.data(), out, got.size() * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy out");
    hip_ok(hipMemcpy(want.data(), ref, want.size() * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy ref");
    double err_prompt = 0, err_decode = 0;
    bool finite = true;
    for (int t = 0; t < total; t++)
        for (long long j = 0; j < orow; j++) {
            const float g = got[(size_t)t * orow + j], w = want[(size_t)t * orow + j];
            if (!std::isfinite(g) || !std::isfinite(w)) finite = false;
            const double d = fabs((double)g - (double)w);
            if (t < o.prompt) err_prompt = d > err_prompt ? d : err_prompt;
            else err_decode = d > err_decode ? d : err_decode;
        }
    if (!o.dump.empty()) {
        std::vector<float> rows((size_t)total * row);
        hip_ok(hipMemcpy(rows.data(), qkv, rows.size() * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy qkv");
        FILE* f = fopen(o.dump.c_str(), "wb");
        if (!f || fwrite(rows.data(), sizeof(float), rows.size(), f) != rows.size() ||
            fwrite(got.data(), sizeof(float), got.size(), f) != got.size() || fclose(f) != 0)
            die("cannot write " + o.dump);
    }
    // (head size 256 over the int8 and 4-bit caches: the split path rounds Q and P to f16 as the reference's
    // attention_decode_tc256 does, against each launch's own running maxima, so a decode step and a verify block
    // of the reference pass agree to about f16's step)
    const double tol_split = hd == 256 && (o.i8 || o.q4) ? 1e-3 : 2e-5;
    // (the f32 kernels' head sizes compute prompts in f32 too: no f16 P)
    const bool f32_path = hd != 64 && hd != 128 && hd != 256;
    const double tol_prompt = o.prompt >= 16 && !f32_path ? 2e-3 : tol_split, tol_decode = tol_split;
    const bool ok = finite && err_prompt <= tol_prompt && err_decode <= tol_decode;
    printf("{\"prompt\": %d, \"steps\": %d, \"heads\": %d, \"kv\": %d, \"hd\": %d, \"cache\": \"%s\", \"graph\": %s, "
           "\"prompt_ms\": %.4f, \"decode_step_us\": %.2f, \"max_abs_prompt\": %.3g, \"max_abs_decode\": %.3g, "
           "\"tol_prompt\": %g, \"tol_decode\": %g, \"ok\": %s}\n",
           o.prompt, o.steps, H, K, hd, o.q4 ? "q4" : o.i8 ? "int8" : "f16", exec ? "true" : "false", prompt_ms,
           o.steps ? 1e3 * step_ms / o.steps : 0.0, err_prompt, err_decode, tol_prompt, tol_decode,
           ok ? "true" : "false");
    fflush(stdout);
    stage("done");
    if (exec) (void)hipGraphExecDestroy(exec);
    return ok ? 0 : 1;
}
