// C ABI of the MI355X backend (include/vestra_hip.h): runtime, tensors,
// prepared projections, Q8_0 tensors and the DA3-BASE block driver.
//
// Each entry point validates every argument before touching HIP, maps HIP
// failures onto the CudaError-shaped status codes and records a thread-local
// message.  Device memory comes from the stream-ordered pool of the
// runtime's device (hipMallocAsync / hipFreeAsync on the runtime stream), so
// chained operators never synchronise and never upload zero-filled buffers
// from the host.
#include "../../include/vestra_hip.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "kernels.h"

#define NEED(p, what) \
    do {              \
        if (!(p)) return null_arg(what); \
    } while (0)

#define TRY(expr)                   \
    do {                            \
        vh_status st_ = (expr);     \
        if (st_ != VH_OK) return st_; \
    } while (0)

#define GUARD_BEGIN try {
#define GUARD_END                                                              \
    }                                                                          \
    catch (const std::bad_alloc &) {                                           \
        return fail(VH_ERR_UPLOAD, "host allocation failed");                 \
    }                                                                          \
    catch (...) {                                                              \
        return fail(VH_ERR_KERNEL, "unexpected host exception");             \
    }

namespace {

thread_local std::string g_err;
thread_local size_t g_mm_dst = 0, g_mm_src = 0;

vh_status fail(vh_status st, const std::string &msg) {
    g_err = msg;
    return st;
}

vh_status mismatch(size_t dst, size_t src, const char *what) {
    g_mm_dst = dst;
    g_mm_src = src;
    return fail(VH_ERR_LENGTH_MISMATCH, std::string(what) + ": length mismatch, destination " +
                                            std::to_string(dst) + ", source " +
                                            std::to_string(src));
}

vh_status null_arg(const char *what) {
    return fail(VH_ERR_INVALID_ARGUMENT, std::string(what) + ": null handle or pointer");
}

std::string hip_msg(const char *what, hipError_t e) {
    return std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
}

struct ProfileRec {
    const char *name;
    hipEvent_t a, b;
};

struct RtState {
    int device = 0;
    hipStream_t stream = nullptr;
    std::mutex mu;
    std::map<std::string, float *> rope_cache;  // host-built sin/cos tables
    float *ws = nullptr;                        // grow-only block workspace
    size_t ws_floats = 0;
    float *sk = nullptr;                        // grow-only split-K partials
    size_t sk_floats = 0;
    float *fw = nullptr;                        // grow-only attention key-split partials
    size_t fw_floats = 0;
    unsigned *fcnt = nullptr;                   // and the in-kernel merge's arrival counters
    size_t fcnt_n = 0;
    char *aq = nullptr;                         // grow-only Q8_0 activation blocks
    size_t aq_bytes = 0;
    float *tw = nullptr;                        // balanced-tail GEMM partials
    unsigned *tcnt = nullptr;                   // and arrival counters (zeroed once)
    float *scratch = nullptr;                   // this device's copy of `scratch` (below)

    bool profile = false;
    std::vector<ProfileRec> pending;
    std::map<std::string, std::pair<unsigned long long, double>> totals;
    hipEvent_t t0 = nullptr, t1 = nullptr;

    ~RtState() {
        if (!stream) return;
        hipSetDevice(device);
        hipStreamSynchronize(stream);
        for (auto &kv : rope_cache) hipFree(kv.second);
        if (ws) hipFree(ws);
        if (sk) hipFree(sk);
        if (fw) hipFree(fw);
        if (fcnt) hipFree(fcnt);
        if (aq) hipFree(aq);
        if (tw) hipFree(tw);
        if (tcnt) hipFree(tcnt);

        for (auto &p : pending) {
            hipEventDestroy(p.a);
            hipEventDestroy(p.b);
        }
        if (t0) hipEventDestroy(t0);
        if (t1) hipEventDestroy(t1);
        hipStreamDestroy(stream);
    }
};

using Rt = std::shared_ptr<RtState>;

}  // namespace

struct vh_runtime {
    Rt s;
};

struct vh_tensor {
    Rt rt;
    float *ptr = nullptr;
    size_t len = 0;
    ~vh_tensor() {
        if (ptr && rt) {
            hipSetDevice(rt->device);
            hipFreeAsync(ptr, rt->stream);
        }
    }
};

namespace {

struct Lin {
    size_t K = 0, N = 0;
    float *wt = nullptr;  // [N][K]
    float *bias = nullptr;
    float *gamma = nullptr;  // null = unit LayerScale
    // Set for a projection that takes a LayerNorm of its input folded in
    // (prepare_lin_ln): wt = W diag(ln gamma), bias = b + W . ln beta and
    // ln_c[n] = sum_k wt[n][k].
    float *ln_c = nullptr;
};

// A projection with Q8_0 weights: W^T [N][K] as block-major blocks,
// qs [K/32][N][32] and d [K/32][N] (binary16 bits).
struct Q8Lin {
    size_t K = 0, N = 0;
    int8_t *qs = nullptr;
    uint16_t *d = nullptr;
    float *bias = nullptr;
    float *gamma = nullptr;  // null = unit LayerScale
    void release(hipStream_t s) {
        if (qs) hipFreeAsync(qs, s);
        if (d) hipFreeAsync(d, s);
        for (float *p : {bias, gamma})
            if (p) hipFreeAsync(p, s);
        *this = Q8Lin{};
    }
};

}  // namespace

struct vh_linear {
    Rt rt;
    Lin L;
    ~vh_linear() {
        if (!rt) return;
        hipSetDevice(rt->device);
        for (float *p : {L.wt, L.bias, L.gamma})
            if (p) hipFreeAsync(p, rt->stream);
    }
};

struct vh_q8_tensor {
    Rt rt;
    size_t rows = 0, k = 0;
    int8_t *qs = nullptr;
    uint16_t *d = nullptr;
    ~vh_q8_tensor() {
        if (!rt) return;
        hipSetDevice(rt->device);
        if (qs) hipFreeAsync(qs, rt->stream);
        if (d) hipFreeAsync(d, rt->stream);
    }
};

struct vh_linear_q8 {
    Rt rt;
    Q8Lin L;
    ~vh_linear_q8() {
        if (!rt) return;
        hipSetDevice(rt->device);
        L.release(rt->stream);
    }
};

struct vh_block {
    Rt rt;
    Lin qkv, proj, fc1, fc2;
    bool q8 = false;  // projections in Q8_0 (qqkv..qfc2) instead of f32
    Q8Lin qqkv, qproj, qfc1, qfc2;
    float *ln1_g = nullptr, *ln1_b = nullptr, *ln2_g = nullptr, *ln2_b = nullptr;
    float *qn_g = nullptr, *qn_b = nullptr, *kn_g = nullptr, *kn_b = nullptr;  // late blocks
    ~vh_block() {
        if (!rt) return;
        hipSetDevice(rt->device);
        for (Lin *l : {&qkv, &proj, &fc1, &fc2})
            for (float *p : {l->wt, l->bias, l->gamma, l->ln_c})
                if (p) hipFreeAsync(p, rt->stream);
        for (Q8Lin *l : {&qqkv, &qproj, &qfc1, &qfc2}) l->release(rt->stream);
        for (float *p : {ln1_g, ln1_b, ln2_g, ln2_b, qn_g, qn_b, kn_g, kn_b})
            if (p) hipFreeAsync(p, rt->stream);
    }
};

namespace {

// ---- device helpers ----------------------------------------------------------

vh_status set_device(RtState &s) {
    hipError_t e = hipSetDevice(s.device);
    if (e != hipSuccess) return fail(VH_ERR_KERNEL, hip_msg("hipSetDevice", e));
    return VH_OK;
}

template <class T>
vh_status dalloc(RtState &s, size_t count, T **out, const char *what) {
    size_t bytes = (count ? count : 1) * sizeof(T);
    void *p = nullptr;
    hipError_t e = hipMallocAsync(&p, bytes, s.stream);
    if (e != hipSuccess) return fail(VH_ERR_UPLOAD, hip_msg(what, e));
    *out = static_cast<T *>(p);
    return VH_OK;
}

vh_status h2d(RtState &s, void *dst, const void *src, size_t bytes, const char *what) {
    if (bytes == 0) return VH_OK;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s.stream);  // host buffer reusable on return
    if (e != hipSuccess) return fail(VH_ERR_UPLOAD, hip_msg(what, e));
    return VH_OK;
}

vh_status upload_array(RtState &s, const float *host, size_t n, float **out, const char *what) {
    vh_status st = dalloc(s, n, out, what);
    if (st) return st;
    st = h2d(s, *out, host, n * sizeof(float), what);
    if (st) {
        hipFreeAsync(*out, s.stream);
        *out = nullptr;
    }
    return st;
}

vh_status new_tensor(const Rt &rt, size_t len, vh_tensor **out, const char *what) {
    float *p = nullptr;
    vh_status st = dalloc(*rt, len, &p, what);
    if (st) return st;
    vh_tensor *t = new (std::nothrow) vh_tensor;
    if (!t) {
        hipFreeAsync(p, rt->stream);
        return fail(VH_ERR_UPLOAD, std::string(what) + ": host allocation failed");
    }
    t->rt = rt;
    t->ptr = p;
    t->len = len;
    *out = t;
    return VH_OK;
}

// Runs a launcher, bracketing it with profiling events when enabled.
template <class F>
vh_status launch(RtState &s, const char *name, F &&f) {
    hipEvent_t a = nullptr, b = nullptr;
    if (s.profile) {
        hipEventCreate(&a);
        hipEventCreate(&b);
        hipEventRecord(a, s.stream);
    }
    hipError_t e = f();
    if (s.profile) {
        hipEventRecord(b, s.stream);
        s.pending.push_back({name, a, b});
    }
    if (e != hipSuccess) return fail(VH_ERR_KERNEL, hip_msg(name, e));
    return VH_OK;
}

// rope::rope2d / rope_rotations tables (src/rope.rs:42-60,
// src/specialized.rs:389-410), built on the host with the platform libm the
// reference calls and cached per (positions, head_dim, frequency).
vh_status rope_table(RtState &s, const int64_t *pos, size_t n, size_t head_dim, float freq,
                     const float **out) {
    const size_t half = head_dim / 2, quarter = half / 2;
    std::string key;
    key.append(reinterpret_cast<const char *>(&freq), sizeof(freq));
    key.append(reinterpret_cast<const char *>(&head_dim), sizeof(head_dim));
    key.append(reinterpret_cast<const char *>(pos), n * 2 * sizeof(int64_t));
    std::lock_guard<std::mutex> lock(s.mu);
    auto it = s.rope_cache.find(key);
    if (it != s.rope_cache.end()) {
        *out = it->second;
        return VH_OK;
    }
    std::vector<float> inv(quarter);
    for (size_t i = 0; i < quarter; i++) inv[i] = powf(freq, -2.0f * (float)i / (float)half);
    std::vector<float> rot(n * 2 * quarter * 2);
    for (size_t p = 0; p < n; p++)
        for (size_t axis = 0; axis < 2; axis++) {
            const float position = (float)pos[2 * p + axis];
            for (size_t i = 0; i < quarter; i++) {
                const float arg = position * inv[i];
                const size_t o = ((p * 2 + axis) * quarter + i) * 2;
                rot[o] = sinf(arg);
                rot[o + 1] = cosf(arg);
            }
        }
    float *d = nullptr;
    hipError_t e = hipMalloc(&d, rot.size() * sizeof(float));
    if (e != hipSuccess) return fail(VH_ERR_UPLOAD, hip_msg("RoPE table allocation", e));
    e = hipMemcpy(d, rot.data(), rot.size() * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        hipFree(d);
        return fail(VH_ERR_UPLOAD, hip_msg("RoPE table upload", e));
    }
    s.rope_cache.emplace(key, d);
    *out = d;
    return VH_OK;
}

vh_status workspace(RtState &s, size_t floats, float **out) {
    if (s.ws_floats < floats) {
        hipStreamSynchronize(s.stream);
        if (s.ws) hipFree(s.ws);
        s.ws = nullptr;
        s.ws_floats = 0;
        hipError_t e = hipMalloc(&s.ws, floats * sizeof(float));
        if (e != hipSuccess) return fail(VH_ERR_UPLOAD, hip_msg("block workspace allocation", e));
        s.ws_floats = floats;
    }
    *out = s.ws;
    return VH_OK;
}

// Split-K partial tiles for the narrow (N <= 1024) projections: up to 8
// splits of an m x n output.
constexpr size_t kMaxSplits = 8;
vh_status splitk_workspace(RtState &s, size_t m, size_t n, float **out, size_t *floats) {
    *out = nullptr;
    *floats = 0;
    if (n > 1024) return VH_OK;
    const size_t need = kMaxSplits * m * n;
    if (s.sk_floats < need) {
        hipStreamSynchronize(s.stream);
        if (s.sk) hipFree(s.sk);
        s.sk = nullptr;
        s.sk_floats = 0;
        hipError_t e = hipMalloc(&s.sk, need * sizeof(float));
        if (e != hipSuccess) return fail(VH_ERR_UPLOAD, hip_msg("split-K workspace allocation", e));
        s.sk_floats = need;
    }
    *out = s.sk;
    *floats = s.sk_floats;
    return VH_OK;
}

// Balanced-tail workspace of the wide GEMMs, allocated on first use.  The
// counters are zeroed once here, on the runtime stream (so ahead of the
// first launch that reads them, which the stream's non-blocking flag would
// not order after a null-stream memset); every launch leaves them zero.
vh_status tail_workspace(RtState &s, vh::GemmArgs &g) {
    if (!s.tw) {
        hipStreamSynchronize(s.stream);
        hipError_t e = hipMalloc(&s.tw, (vh::kTailFloats + vh::kTailStatFloats) * sizeof(float));
        if (e == hipSuccess) e = hipMalloc(&s.tcnt, vh::kTailTiles * sizeof(unsigned));
        if (e == hipSuccess) e = hipMemsetAsync(s.tcnt, 0, vh::kTailTiles * sizeof(unsigned), s.stream);
        if (e != hipSuccess) {
            if (s.tw) hipFree(s.tw);
            if (s.tcnt) hipFree(s.tcnt);
            s.tw = nullptr;
            s.tcnt = nullptr;
            return fail(VH_ERR_UPLOAD, hip_msg("GEMM tail workspace allocation", e));
        }
    }
    g.tail_ws = s.tw;
    g.tail_ws_floats = vh::kTailFloats;
    g.tail_stats = s.tw + vh::kTailFloats;
    g.tail_cnt = s.tcnt;
    g.tail_cnt_n = vh::kTailTiles;
    return VH_OK;
}

// The flash grid holds heads * ceil(tokens/64) * splits workgroups of 256
// threads; its thread count must fit the 32-bit launch limit.
bool flash_grid_fits(size_t heads, size_t tokens) {
    const size_t qtiles = (tokens + 63) / 64;
    size_t items = 0;
    return !__builtin_mul_overflow(heads, qtiles, &items) &&
           items <= (size_t)UINT32_MAX / 256 / vh::kMaxFlashSplits;
}

vh_status flash(RtState &s, const float *q, const float *k, const float *v, float *out,
                size_t bh, size_t tokens, size_t heads, bool token_major, int8_t *q8_qs = nullptr,
                uint16_t *q8_d = nullptr, bool *quantized = nullptr, float scale = 0.125f) {
    // Partials of the key splits (room for either layout: the merge launch's
    // or the in-kernel merge's); without them the kernel runs unsplit.
    const size_t need =
        std::max(vh::flash_workspace_floats(bh, tokens), vh::flash_fused_workspace_floats(bh, tokens));
    if (s.fw_floats < need) {
        hipStreamSynchronize(s.stream);
        if (s.fw) hipFree(s.fw);
        s.fw = nullptr;
        s.fw_floats = 0;
        if (hipMalloc(&s.fw, need * sizeof(float)) == hipSuccess) s.fw_floats = need;
        else hipGetLastError();
    }
    // Arrival counters of the in-kernel merge, zeroed once here (outside any
    // stream capture: the first run of a shape allocates); every run leaves
    // them zero.  Without them the merge runs as its own launch.
    const size_t groups = vh::flash_query_groups(bh, tokens);
    if (s.fcnt_n < groups) {
        hipStreamSynchronize(s.stream);
        if (s.fcnt) hipFree(s.fcnt);
        s.fcnt = nullptr;
        s.fcnt_n = 0;
        if (hipMalloc(&s.fcnt, groups * sizeof(unsigned)) == hipSuccess &&
            hipMemsetAsync(s.fcnt, 0, groups * sizeof(unsigned), s.stream) == hipSuccess) {
            s.fcnt_n = groups;
        } else {
            hipGetLastError();
            if (s.fcnt) hipFree(s.fcnt);
            s.fcnt = nullptr;
        }
    }
    return launch(s, "flash_attention", [&] {
        return vh::launch_flash_attention(s.stream, q, k, v, out, bh, tokens, heads, token_major,
                                          s.fw, s.fw_floats, q8_qs, q8_d, quantized, scale, s.fcnt,
                                          s.fcnt_n);
    });
}

vh_status prepare_lin(RtState &s, size_t K, size_t N, const float *w, const float *bias,
                      const float *gamma, Lin *L) {
    float *tmp = nullptr;
    vh_status st = upload_array(s, w, K * N, &tmp, "linear weight upload");
    if (st) return st;
    st = dalloc(s, K * N, &L->wt, "linear weight allocation");
    if (!st)
        st = launch(s, "transpose_weight", [&] { return vh::launch_transpose(s.stream, tmp, L->wt, K, N); });
    hipFreeAsync(tmp, s.stream);
    if (!st) st = upload_array(s, bias, N, &L->bias, "linear bias upload");
    if (!st && gamma) st = upload_array(s, gamma, N, &L->gamma, "linear gamma upload");
    if (st) {
        for (float *p : {L->wt, L->bias, L->gamma})
            if (p) hipFreeAsync(p, s.stream);
        *L = Lin{};
        return st;
    }
    L->K = K;
    L->N = N;
    return VH_OK;
}

// A projection of LayerNorm(x) (gamma g, beta be) prepared for the folded
// form LayerNorm(x) . W^T + b = rstd * (x . W'^T - mean * c) + b' (see
// GemmArgs::ln_fold_c): W'[n][k] = W[k][n] * g[k] (w is [K][N], in x out),
// c[n] = sum_k W'[n][k] and b'[n] = b[n] + sum_k W[k][n] * be[k], both sums in
// double over the rounded W' and the given W.
vh_status prepare_lin_ln(RtState &s, size_t K, size_t N, const float *w, const float *bias,
                         const float *ln_g, const float *ln_b, Lin *L) {
    if (!w || !bias || !ln_g || !ln_b) return null_arg("prepare_lin_ln");
    std::vector<float> wt(K * N), c(N), bp(N);
    for (size_t n = 0; n < N; n++) {
        double cs = 0.0, bs = (double)bias[n];
        for (size_t k = 0; k < K; k++) {
            const float wv = w[k * N + n];
            const float f = wv * ln_g[k];
            wt[n * K + k] = f;
            cs += (double)f;
            bs += (double)wv * (double)ln_b[k];
        }
        c[n] = (float)cs;
        bp[n] = (float)bs;
    }
    vh_status st = upload_array(s, wt.data(), K * N, &L->wt, "linear weight upload");
    if (!st) st = upload_array(s, bp.data(), N, &L->bias, "linear bias upload");
    if (!st) st = upload_array(s, c.data(), N, &L->ln_c, "linear LayerNorm fold upload");
    if (st) {
        for (float *p : {L->wt, L->bias, L->ln_c})
            if (p) hipFreeAsync(p, s.stream);
        *L = Lin{};
        return st;
    }
    L->K = K;
    L->N = N;
    return VH_OK;
}

// LayerNorm applied to the rows a Residual GEMM has just updated.
struct RowNorm {
    const float *gamma, *beta;
    float *out;
    float eps;
};

// Row statistics passed between a Residual GEMM and the LayerNorm-folded
// GEMM after it: (mean, M2) per column chunk of each row (GemmArgs).
struct ChunkStats {
    const float *in = nullptr;     // the input rows' statistics, or null
    size_t in_chunks = 0;          // chunks per row of in
    float *out = nullptr;          // where a Residual GEMM writes them, or null
    int *out_chunks = nullptr;     // chunks per row written to out (0: none)
};

vh_status run_lin(RtState &s, const Lin &L, const float *in, size_t rows, vh::Epi epi, float *c,
                  const char *name, const RowNorm *norm = nullptr, float fold_eps = 0.0f,
                  const ChunkStats &cs = ChunkStats{}) {
    vh::GemmArgs g{};
    g.a = in;
    g.bt = L.wt;
    g.m = rows;
    g.n = L.N;
    g.k = L.K;
    g.epi = epi;
    g.c = c;
    g.bias = L.bias;
    g.gamma = epi == vh::Epi::Gelu ? nullptr : L.gamma;
    if (norm) {
        g.ln_gamma = norm->gamma;
        g.ln_beta = norm->beta;
        g.ln_out = norm->out;
        g.ln_eps = norm->eps;
    }
    g.ln_fold_c = L.ln_c;
    g.ln_fold_eps = fold_eps;
    if (cs.in && cs.in_chunks) {
        g.stats_in = cs.in;
        g.stats_in_chunks = cs.in_chunks;
    }
    if (cs.out) {
        g.stats_out = cs.out;
        g.stats_out_chunks = cs.out_chunks;
    }
    TRY(splitk_workspace(s, rows, L.N, &g.ws, &g.ws_floats));
    TRY(tail_workspace(s, g));
    return launch(s, name, [&] { return vh::launch_gemm(s.stream, g); });
}

vh_status run_qkv(RtState &s, const Lin &L, const float *in, size_t images, size_t tokens,
                  size_t heads, const float *rot, float *q, float *k, float *v, float fold_eps = 0.0f,
                  const float *stats_in = nullptr, size_t stats_in_chunks = 0) {
    vh::GemmArgs g{};
    g.ln_fold_c = L.ln_c;
    g.ln_fold_eps = fold_eps;
    if (stats_in && stats_in_chunks) {
        g.stats_in = stats_in;
        g.stats_in_chunks = stats_in_chunks;
    }
    g.a = in;
    g.bt = L.wt;
    g.m = images * tokens;
    g.n = L.N;
    g.k = L.K;
    g.epi = vh::Epi::Qkv;
    g.bias = L.bias;
    g.q = q;
    g.k_out = k;
    g.v = v;
    g.tokens = tokens;
    g.heads = heads;
    g.rot = rot;
    return launch(s, "gemm_qkv_rope", [&] { return vh::launch_gemm(s.stream, g); });
}

bool mul_overflows(size_t a, size_t b, size_t *out) { return __builtin_mul_overflow(a, b, out); }

// Block-major Q8_0 blocks of a rows x k activation: qs, then d 256 bytes on.
vh_status q8_workspace(RtState &s, size_t rows, size_t k, int8_t **qs, uint16_t **d) {
    const size_t qbytes = (rows * k + 255) & ~size_t(255);
    const size_t need = qbytes + rows * (k / 32) * sizeof(uint16_t);
    if (s.aq_bytes < need) {
        hipStreamSynchronize(s.stream);
        if (s.aq) hipFree(s.aq);
        s.aq = nullptr;
        s.aq_bytes = 0;
        hipError_t e = hipMalloc(&s.aq, need);
        if (e != hipSuccess) return fail(VH_ERR_UPLOAD, hip_msg("Q8_0 activation workspace allocation", e));
        s.aq_bytes = need;
    }
    *qs = reinterpret_cast<int8_t *>(s.aq);
    *d = reinterpret_cast<uint16_t *>(s.aq + qbytes);
    return VH_OK;
}

// Q8_0 activation rows in the runtime workspace: quantize_row_q8_0 of `in`,
// or, with norm, the LayerNorm of `in` quantised in the same kernel.
struct Q8Rows {
    int8_t *qs = nullptr;
    uint16_t *d = nullptr;
};
vh_status q8_rows(RtState &s, const float *in, size_t rows, size_t k, const RowNorm *norm,
                  Q8Rows *out) {
    TRY(q8_workspace(s, rows, k, &out->qs, &out->d));
    if (norm)
        return launch(s, "layernorm_q8_0", [&] {
            return vh::launch_layernorm_q8_0(s.stream, in, norm->gamma, norm->beta, out->qs,
                                             out->d, rows, k, norm->eps);
        });
    return launch(s, "quantize_q8_0", [&] {
        return vh::launch_quantize_q8_0(s.stream, in, out->qs, out->d, rows, k);
    });
}

// The engine's Q8_0 projection: quantise the input rows (quantize_row_q8_0;
// with norm, of LayerNorm(in)), block-dot GEMM against the weight blocks,
// then the epilogue.
vh_status run_q8(RtState &s, const Q8Lin &L, const float *in, size_t rows, vh::Epi epi, float *c,
                 const char *name, const RowNorm *norm = nullptr) {
    Q8Rows a;
    TRY(q8_rows(s, in, rows, L.K, norm, &a));
    return launch(s, name, [&] {
        return vh::launch_gemm_q8_0(s.stream, a.qs, a.d, L.qs, L.d, c, rows, L.N, L.K, epi, L.bias,
                                    epi == vh::Epi::Gelu ? nullptr : L.gamma);
    });
}

// The QKV projection in Q8_0, written head-major with the RoPE when rot is set.
vh_status run_q8_qkv(RtState &s, const Q8Lin &L, const float *in, size_t images, size_t tokens,
                     const float *rot, float *q, float *k, float *v, const RowNorm *norm = nullptr) {
    const size_t rows = images * tokens;
    Q8Rows a;
    TRY(q8_rows(s, in, rows, L.K, norm, &a));
    int8_t *qs = a.qs;
    uint16_t *d = a.d;
    return launch(s, "gemm_q8_0_qkv", [&] {
        return vh::launch_gemm_q8_0_qkv(s.stream, qs, d, L.qs, L.d, rows, L.K, L.bias, q, k, v,
                                        tokens, L.N / 192, rot);
    });
}

// f32 weights [K][N] row-major -> Q8_0 blocks of W^T rows, quantised on the
// device with the activation kernel (quantize_row_q8_0 of each column).
vh_status prepare_q8_from_f32(RtState &s, size_t K, size_t N, const float *w, const float *bias,
                              const float *gamma, Q8Lin *Q) {
    Lin L;
    TRY(prepare_lin(s, K, N, w, bias, gamma, &L));
    vh_status st = dalloc(s, K * N, &Q->qs, "Q8_0 weight allocation");
    if (!st) st = dalloc(s, N * (K / 32), &Q->d, "Q8_0 weight allocation");
    if (!st)
        st = launch(s, "quantize_q8_0", [&] {
            return vh::launch_quantize_q8_0(s.stream, L.wt, Q->qs, Q->d, N, K);
        });
    hipFreeAsync(L.wt, s.stream);
    Q->bias = L.bias;
    Q->gamma = L.gamma;
    if (st) {
        Q->release(s.stream);
        return st;
    }
    Q->K = K;
    Q->N = N;
    return VH_OK;
}

}  // namespace

// =============================================================================
// no-allocation scratch
// =============================================================================

// Key-split partials of vh_flash_attention_f32_da3_base_into: a file-scope
// device array, one copy per GPU, held until the process ends.  Host code
// never passes `scratch` itself (on the host the name is only a stand-in);
// it passes the device address hipGetSymbolAddress returned for the current
// device, cached per device by scratch_init.
constexpr size_t kScratchBytes = size_t(64) << 20;
constexpr size_t kScratchFloats = kScratchBytes / sizeof(float);
static __device__ __align__(256) float scratch[kScratchFloats];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;  // guards the slots and orders the uses of each array
float *g_scratch_ptr[kMaxScratchDevices] = {};
// Per device, an event recorded after the last launch that used its array,
// on whichever stream it ran: the next use, from any stream, waits for it.
// Created with the slot, never destroyed (the array also lives until exit).
hipEvent_t g_scratch_done[kMaxScratchDevices] = {};

// With `device` current: its address of `scratch` and its last-use event,
// set up once.
vh_status scratch_init(int device, float **out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || device >= kMaxScratchDevices)
        return fail(VH_ERR_INITIALIZE, "no scratch slot for HIP device " + std::to_string(device));
    if (!g_scratch_ptr[device]) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(VH_ERR_INITIALIZE, hip_msg("scratch symbol address", e));
        hipEvent_t ev = nullptr;
        e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) return fail(VH_ERR_INITIALIZE, hip_msg("scratch event", e));
        g_scratch_done[device] = ev;
        g_scratch_ptr[device] = static_cast<float *>(p);
    }
    *out = g_scratch_ptr[device];
    return VH_OK;
}

}  // namespace

// =============================================================================
// errors
// =============================================================================

extern "C" const char *vh_last_error(void) { return g_err.c_str(); }

extern "C" void vh_last_length_mismatch(size_t *destination, size_t *source_len) {
    if (destination) *destination = g_mm_dst;
    if (source_len) *source_len = g_mm_src;
}

// =============================================================================
// runtime
// =============================================================================

extern "C" vh_status vh_runtime_new(size_t device, vh_runtime **out) {
    NEED(out, "vh_runtime_new");
    GUARD_BEGIN
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0)
        return fail(VH_ERR_INITIALIZE, "failed to initialize HIP device " + std::to_string(device) +
                                           ": no HIP device (" + hipGetErrorString(e) + ")");
    if (device >= (size_t)count)
        return fail(VH_ERR_INITIALIZE, "failed to initialize HIP device " + std::to_string(device) +
                                           ": only " + std::to_string(count) + " device(s)");
    auto s = std::make_shared<RtState>();
    s->device = (int)device;
    e = hipSetDevice(s->device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
    if (e != hipSuccess)
        return fail(VH_ERR_INITIALIZE, "failed to initialize HIP device " + std::to_string(device) +
                                           ": " + hipGetErrorString(e));
    TRY(scratch_init(s->device, &s->scratch));
    // Keep freed blocks in the stream-ordered pool instead of returning them
    // to the driver at every synchronisation.
    hipMemPool_t pool = nullptr;
    if (hipDeviceGetDefaultMemPool(&pool, s->device) == hipSuccess && pool) {
        uint64_t threshold = UINT64_MAX;
        hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &threshold);
    }
    vh_runtime *rt = new vh_runtime;
    rt->s = s;
    *out = rt;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_runtime_clone(const vh_runtime *rt, vh_runtime **out) {
    NEED(rt, "vh_runtime_clone");
    NEED(out, "vh_runtime_clone");
    GUARD_BEGIN
    vh_runtime *c = new vh_runtime;
    c->s = rt->s;
    *out = c;
    return VH_OK;
    GUARD_END
}

extern "C" void vh_runtime_free(vh_runtime *rt) { delete rt; }

extern "C" size_t vh_runtime_device(const vh_runtime *rt) { return rt ? (size_t)rt->s->device : 0; }

extern "C" void *vh_runtime_stream(const vh_runtime *rt) {
    return rt ? (void *)rt->s->stream : nullptr;
}

extern "C" vh_status vh_runtime_synchronize(const vh_runtime *rt) {
    NEED(rt, "vh_runtime_synchronize");
    TRY(set_device(*rt->s));
    hipError_t e = hipStreamSynchronize(rt->s->stream);
    if (e != hipSuccess) return fail(VH_ERR_KERNEL, hip_msg("stream synchronize", e));
    return VH_OK;
}

// =============================================================================
// tensors
// =============================================================================

extern "C" vh_status vh_upload_f32(const vh_runtime *rt, const float *values, size_t len,
                                   vh_tensor **out) {
    NEED(rt, "vh_upload_f32");
    NEED(out, "vh_upload_f32");
    if (len && !values) return null_arg("vh_upload_f32 values");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, len, &t, "upload allocation"));
    vh_status st = h2d(s, t->ptr, values, len * sizeof(float), "host-to-device transfer");
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_download_f32(const vh_runtime *rt, const vh_tensor *tensor, float *out,
                                     size_t out_len) {
    NEED(rt, "vh_download_f32");
    NEED(tensor, "vh_download_f32");
    if (out_len != tensor->len) return mismatch(out_len, tensor->len, "vh_download_f32");
    if (out_len && !out) return null_arg("vh_download_f32 out");
    RtState &s = *rt->s;
    TRY(set_device(s));
    if (out_len == 0) return VH_OK;
    hipError_t e = hipMemcpyAsync(out, tensor->ptr, out_len * sizeof(float),
                                  hipMemcpyDeviceToHost, s.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s.stream);
    if (e != hipSuccess) return fail(VH_ERR_DOWNLOAD, hip_msg("device-to-host transfer", e));
    return VH_OK;
}

extern "C" vh_status vh_tensor_alloc(const vh_runtime *rt, size_t len, vh_tensor **out) {
    NEED(rt, "vh_tensor_alloc");
    NEED(out, "vh_tensor_alloc");
    GUARD_BEGIN
    TRY(set_device(*rt->s));
    return new_tensor(rt->s, len, out, "tensor allocation");
    GUARD_END
}

extern "C" void vh_tensor_free(vh_tensor *tensor) { delete tensor; }
extern "C" size_t vh_tensor_len(const vh_tensor *tensor) { return tensor ? tensor->len : 0; }
extern "C" int vh_tensor_is_empty(const vh_tensor *tensor) { return !tensor || tensor->len == 0; }
extern "C" float *vh_tensor_device_ptr(const vh_tensor *tensor) {
    return tensor ? tensor->ptr : nullptr;
}

// =============================================================================
// copies / residual
// =============================================================================

// Device copies: the streaming copy kernel for large 16-byte-aligned runs
// (non-temporal, faster than the runtime's copy engine path), else
// hipMemcpyAsync.
static vh_status d2d(RtState &s, float *dst, const float *src, size_t n, const char *what) {
    if (n == 0) return VH_OK;
    return launch(s, what, [&] {
        if (vh::stream_copy_applies(dst, src, n)) return vh::launch_stream_copy(s.stream, dst, src, n);
        return hipMemcpyAsync(dst, src, n * sizeof(float), hipMemcpyDeviceToDevice, s.stream);
    });
}

extern "C" vh_status vh_copy_f32(const vh_runtime *rt, const vh_tensor *source, vh_tensor **out) {
    NEED(rt, "vh_copy_f32");
    NEED(source, "vh_copy_f32");
    NEED(out, "vh_copy_f32");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, source->len, &t, "copy allocation"));
    vh_status st = d2d(s, t->ptr, source->ptr, source->len, "copy");
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_copy_segment_f32(const vh_runtime *rt, const vh_tensor *source,
                                         size_t source_offset, size_t len, vh_tensor **out) {
    NEED(rt, "vh_copy_segment_f32");
    NEED(source, "vh_copy_segment_f32");
    NEED(out, "vh_copy_segment_f32");
    size_t end = 0;
    if (__builtin_add_overflow(source_offset, len, &end) || end > source->len)
        return mismatch(len, source->len > source_offset ? source->len - source_offset : 0,
                        "vh_copy_segment_f32");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, len, &t, "segment allocation"));
    vh_status st = d2d(s, t->ptr, source->ptr + source_offset, len, "copy_segment");
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_copy_segment_into_f32(const vh_runtime *rt, vh_tensor *destination,
                                              size_t destination_offset, const vh_tensor *source,
                                              size_t source_offset, size_t len) {
    NEED(rt, "vh_copy_segment_into_f32");
    NEED(destination, "vh_copy_segment_into_f32");
    NEED(source, "vh_copy_segment_into_f32");
    size_t dend = 0, send = 0;
    bool bad = __builtin_add_overflow(destination_offset, len, &dend) ||
               __builtin_add_overflow(source_offset, len, &send) || dend > destination->len ||
               send > source->len;
    if (bad)
        return mismatch(destination->len > destination_offset ? destination->len - destination_offset : 0,
                        source->len > source_offset ? source->len - source_offset : 0,
                        "vh_copy_segment_into_f32");
    RtState &s = *rt->s;
    TRY(set_device(s));
    return d2d(s, destination->ptr + destination_offset, source->ptr + source_offset, len,
               "copy_segment_into");
}

extern "C" vh_status vh_overwrite_prefix_f32(const vh_runtime *rt, vh_tensor *destination,
                                             const vh_tensor *source, size_t len) {
    NEED(rt, "vh_overwrite_prefix_f32");
    NEED(destination, "vh_overwrite_prefix_f32");
    NEED(source, "vh_overwrite_prefix_f32");
    if (len > destination->len || len > source->len)
        return mismatch(destination->len, source->len, "vh_overwrite_prefix_f32");
    RtState &s = *rt->s;
    TRY(set_device(s));
    return d2d(s, destination->ptr, source->ptr, len, "overwrite_prefix");
}

extern "C" vh_status vh_add_f32_in_place(const vh_runtime *rt, vh_tensor *destination,
                                         const vh_tensor *source) {
    NEED(rt, "vh_add_f32_in_place");
    NEED(destination, "vh_add_f32_in_place");
    NEED(source, "vh_add_f32_in_place");
    if (destination->len != source->len)
        return mismatch(destination->len, source->len, "vh_add_f32_in_place");
    RtState &s = *rt->s;
    TRY(set_device(s));
    return launch(s, "add", [&] {
        return vh::launch_add(s.stream, destination->ptr, source->ptr, destination->len);
    });
}

// =============================================================================
// GEMM and epilogues
// =============================================================================

extern "C" vh_status vh_gemm_row_major_f32(const vh_runtime *rt, const vh_tensor *a,
                                           const vh_tensor *b, size_t m, size_t k, size_t n,
                                           vh_tensor **out) {
    NEED(rt, "vh_gemm_row_major_f32");
    NEED(a, "vh_gemm_row_major_f32");
    NEED(b, "vh_gemm_row_major_f32");
    NEED(out, "vh_gemm_row_major_f32");
    size_t mk = 0, kn = 0, mn = 0;
    if (mul_overflows(m, k, &mk) || mul_overflows(k, n, &kn) || mul_overflows(m, n, &mn) ||
        a->len != mk || b->len != kn)
        return fail(VH_ERR_BLAS, "row-major GEMM shape M=" + std::to_string(m) + ", K=" +
                                     std::to_string(k) + ", N=" + std::to_string(n) +
                                     " does not match A=" + std::to_string(a->len) +
                                     " or B=" + std::to_string(b->len));
    if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
        return fail(VH_ERR_BLAS, "row-major GEMM dimension exceeds 2^31-1");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, mn, &t, "GEMM output allocation"));
    // B read in place, K-major: the direct convolution's loader as a 1 x 1
    // tap over a one-row "image" of n pixels and k channels, whose
    // channel-major output is row-major C; no transposed copy of B.  Its
    // eight 4-byte loads per thread and slice cost what the copy saves at
    // M, K <= 1024 (per-launch events, 865 x 768 x 3072: 49.2 us against 39.3
    // + 10.4 for the copy and the NT GEMM; per call, with the copy's
    // allocation, 47.5 against 101.5 us), and lose beyond (865 x 3072 x 768
    // 54.2 against 50.8, 3460 x 768 x 3072 167 against 140, 4096^3 1286
    // against 1009).  VESTRA_HIP_GEMM_RM_DIRECT=0|1 forces either route.
    const char *rm_env = std::getenv("VESTRA_HIP_GEMM_RM_DIRECT");
    const bool rm_direct = rm_env ? rm_env[0] != '0' : (m <= 1024 && k <= 1024);
    if (k > 0 && k % 32 == 0 && rm_direct) {
        vh::GemmArgs g{};
        g.a = a->ptr;
        g.bt = b->ptr;
        g.m = m;
        g.n = n;
        g.k = k;
        g.epi = vh::Epi::Store;
        g.c = t->ptr;
        g.conv_in_c = k;
        g.conv_kw = 1;
        g.conv_ow = n;
        g.conv_ih = 1;
        g.conv_iw = n;
        g.conv_stride = 1;
        vh_status st = tail_workspace(s, g);
        if (!st) st = launch(s, "gemm", [&] { return vh::launch_gemm(s.stream, g); });
        if (st) {
            delete t;
            return st;
        }
        *out = t;
        return VH_OK;
    }
    float *bt = nullptr;
    vh_status st = dalloc(s, kn, &bt, "GEMM operand allocation");
    if (!st)
        st = launch(s, "transpose_b", [&] { return vh::launch_transpose(s.stream, b->ptr, bt, k, n); });
    if (!st) {
        vh::GemmArgs g{};
        g.a = a->ptr;
        g.bt = bt;
        g.m = m;
        g.n = n;
        g.k = k;
        g.epi = vh::Epi::Store;
        g.c = t->ptr;
        st = tail_workspace(s, g);
        if (!st) st = launch(s, "gemm", [&] { return vh::launch_gemm(s.stream, g); });
    }
    if (bt) hipFreeAsync(bt, s.stream);
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_bias_scale_f32_in_place(const vh_runtime *rt, vh_tensor *values,
                                                const vh_tensor *bias, const vh_tensor *gamma,
                                                size_t rows, size_t columns) {
    NEED(rt, "vh_bias_scale_f32_in_place");
    NEED(values, "vh_bias_scale_f32_in_place");
    NEED(bias, "vh_bias_scale_f32_in_place");
    NEED(gamma, "vh_bias_scale_f32_in_place");
    size_t expected = 0;
    if (mul_overflows(rows, columns, &expected) || values->len != expected ||
        bias->len != columns || gamma->len != columns)
        return mismatch(values->len, expected, "vh_bias_scale_f32_in_place");
    RtState &s = *rt->s;
    TRY(set_device(s));
    return launch(s, "bias_scale", [&] {
        return vh::launch_bias_scale(s.stream, values->ptr, bias->ptr, gamma->ptr, rows, columns);
    });
}

extern "C" vh_status vh_gelu_f32_in_place(const vh_runtime *rt, vh_tensor *values) {
    NEED(rt, "vh_gelu_f32_in_place");
    NEED(values, "vh_gelu_f32_in_place");
    RtState &s = *rt->s;
    TRY(set_device(s));
    return launch(s, "gelu", [&] { return vh::launch_gelu(s.stream, values->ptr, values->len); });
}

// =============================================================================
// LayerNorm
// =============================================================================

static vh_status layernorm_common(const vh_runtime *rt, const vh_tensor *input,
                                  const vh_tensor *gamma, const vh_tensor *beta, size_t rows,
                                  size_t columns, float eps, vh_tensor **out, bool cpu_order) {
    const char *name = cpu_order ? "vh_layernorm_f32_cpu_order" : "vh_layernorm_f32";
    NEED(rt, name);
    NEED(input, name);
    NEED(gamma, name);
    NEED(beta, name);
    NEED(out, name);
    size_t expected = 0;
    if (mul_overflows(rows, columns, &expected) || input->len != expected ||
        gamma->len != columns || beta->len != columns)
        return mismatch(input->len, expected, name);
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, expected, &t, "LayerNorm output allocation"));
    vh_status st = launch(s, cpu_order ? "layernorm_cpu_order" : "layernorm", [&] {
        return cpu_order ? vh::launch_layernorm_cpu_order(s.stream, input->ptr, gamma->ptr,
                                                          beta->ptr, t->ptr, rows, columns, eps)
                         : vh::launch_layernorm(s.stream, input->ptr, gamma->ptr, beta->ptr,
                                                t->ptr, rows, columns, eps);
    });
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_layernorm_f32(const vh_runtime *rt, const vh_tensor *input,
                                      const vh_tensor *gamma, const vh_tensor *beta, size_t rows,
                                      size_t columns, float epsilon, vh_tensor **out) {
    return layernorm_common(rt, input, gamma, beta, rows, columns, epsilon, out, false);
}

extern "C" vh_status vh_layernorm_f32_cpu_order(const vh_runtime *rt, const vh_tensor *input,
                                                const vh_tensor *gamma, const vh_tensor *beta,
                                                size_t rows, size_t columns, float epsilon,
                                                vh_tensor **out) {
    return layernorm_common(rt, input, gamma, beta, rows, columns, epsilon, out, true);
}

// =============================================================================
// attention
// =============================================================================

extern "C" vh_status vh_attention_online_f32(const vh_runtime *rt, const vh_tensor *q,
                                             const vh_tensor *k, const vh_tensor *v, size_t heads,
                                             size_t tokens, size_t head_dim, vh_tensor **out) {
    NEED(rt, "vh_attention_online_f32");
    NEED(q, "vh_attention_online_f32");
    NEED(k, "vh_attention_online_f32");
    NEED(v, "vh_attention_online_f32");
    NEED(out, "vh_attention_online_f32");
    if (head_dim == 0 || head_dim > 64)
        return fail(VH_ERR_KERNEL, "online attention supports 1..=64 head dimensions, got " +
                                       std::to_string(head_dim));
    size_t ht = 0, expected = 0;
    if (mul_overflows(heads, tokens, &ht) || mul_overflows(ht, head_dim, &expected) ||
        q->len != expected || k->len != expected || v->len != expected)
        return mismatch(q->len, expected, "vh_attention_online_f32");
    if (tokens > INT32_MAX || ht > INT32_MAX || !flash_grid_fits(heads, tokens))
        return fail(VH_ERR_KERNEL, "attention shape exceeds the launch grid");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, expected, &t, "attention output allocation"));
    vh_status st;
    if (head_dim == 64) {
        st = flash(s, q->ptr, k->ptr, v->ptr, t->ptr, heads, tokens, heads, false);
    } else {
        // Rows zero-padded to 64 dims run through the flash kernel with the
        // 1/sqrt(head_dim) scale; the output keeps the first head_dim columns.
        const size_t padded = ht * 64;
        float *pad = nullptr;
        st = dalloc(s, 4 * padded, &pad, "attention padding allocation");
        if (!st) {
            float *pq = pad, *pk = pad + padded, *pv = pad + 2 * padded, *po = pad + 3 * padded;
            st = launch(s, "attention_pad", [&] {
                return vh::launch_pad_rows64(s.stream, q->ptr, k->ptr, v->ptr, pq, pk, pv, ht,
                                             head_dim);
            });
            if (!st)
                st = flash(s, pq, pk, pv, po, heads, tokens, heads, false, nullptr, nullptr,
                           nullptr, 1.0f / sqrtf((float)head_dim));
            if (!st)
                st = launch(s, "attention_unpad", [&] {
                    return vh::launch_unpad_rows(s.stream, po, t->ptr, ht, head_dim);
                });
            hipFreeAsync(pad, s.stream);
        }
    }
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_flash_attention_f32_da3_base(const vh_runtime *rt, const vh_tensor *q,
                                                     const vh_tensor *k, const vh_tensor *v,
                                                     size_t heads, size_t tokens, int token_major,
                                                     vh_tensor **out) {
    NEED(rt, "vh_flash_attention_f32_da3_base");
    NEED(q, "vh_flash_attention_f32_da3_base");
    NEED(k, "vh_flash_attention_f32_da3_base");
    NEED(v, "vh_flash_attention_f32_da3_base");
    NEED(out, "vh_flash_attention_f32_da3_base");
    size_t ht = 0, expected = 0;
    if (mul_overflows(heads, tokens, &ht) || mul_overflows(ht, 64, &expected) ||
        q->len != expected || k->len != expected || v->len != expected)
        return mismatch(q->len, expected, "vh_flash_attention_f32_da3_base");
    if (tokens > INT32_MAX || heads > 65535 || !flash_grid_fits(heads, tokens))
        return fail(VH_ERR_KERNEL, "flash attention shape exceeds the launch grid");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, expected, &t, "attention output allocation"));
    vh_status st = flash(s, q->ptr, k->ptr, v->ptr, t->ptr, heads, tokens, heads, token_major != 0);
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_flash_attention_f32_da3_base_into(const vh_runtime *rt,
                                                          const vh_tensor *q, const vh_tensor *k,
                                                          const vh_tensor *v, size_t heads,
                                                          size_t tokens, int token_major,
                                                          vh_tensor *out) {
    const char *what = "vh_flash_attention_f32_da3_base_into";
    NEED(rt, what);
    NEED(q, what);
    NEED(k, what);
    NEED(v, what);
    NEED(out, what);
    size_t ht = 0, expected = 0;
    if (mul_overflows(heads, tokens, &ht) || mul_overflows(ht, 64, &expected) ||
        q->len != expected || k->len != expected || v->len != expected)
        return mismatch(q->len, expected, what);
    if (out->len != expected) return mismatch(out->len, expected, what);
    if (tokens > INT32_MAX || heads > 65535 || !flash_grid_fits(heads, tokens))
        return fail(VH_ERR_KERNEL, "flash attention shape exceeds the launch grid");
    // Room for the partials of the largest key split the launcher may pick,
    // so that it picks the split the allocating entry point picks.
    const size_t max_rows = kScratchFloats / vh::flash_workspace_floats(1, 1);
    if (ht > max_rows)
        return fail(VH_ERR_KERNEL, std::string(what) + ": heads*tokens = " + std::to_string(ht) +
                                       " exceeds the no-allocation limit of " +
                                       std::to_string(max_rows) + " (64 MiB of key-split partials)");
    if (heads * tokens == 0) return VH_OK;
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    if (!s.scratch) return fail(VH_ERR_INITIALIZE, std::string(what) + ": no scratch on this device");
    // One use of the device's array at a time, in call order: this stream
    // waits for the last use (on any stream), and this launch becomes the
    // last use.  Under stream capture the graph's own order applies instead
    // (an event recorded outside a capture cannot be waited on inside it).
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    const hipEvent_t done = g_scratch_done[s.device];
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s.stream, &capture);
    if (e != hipSuccess) return fail(VH_ERR_KERNEL, hip_msg(what, e));
    const bool order = capture == hipStreamCaptureStatusNone;
    if (order && (e = hipStreamWaitEvent(s.stream, done, 0)) != hipSuccess)
        return fail(VH_ERR_KERNEL, hip_msg(what, e));
    e = vh::launch_flash_attention(s.stream, q->ptr, k->ptr, v->ptr, out->ptr, heads, tokens, heads,
                                   token_major != 0, s.scratch, kScratchFloats);
    if (e != hipSuccess) return fail(VH_ERR_KERNEL, hip_msg(what, e));
    if (order && (e = hipEventRecord(done, s.stream)) != hipSuccess)
        return fail(VH_ERR_KERNEL, hip_msg(what, e));
    return VH_OK;
    GUARD_END
}

// =============================================================================
// layout
// =============================================================================

extern "C" vh_status vh_split_qkv_hnd_f32(const vh_runtime *rt, const vh_tensor *qkv,
                                          size_t tokens, size_t heads, size_t head_dim,
                                          vh_tensor **q, vh_tensor **k, vh_tensor **v) {
    NEED(rt, "vh_split_qkv_hnd_f32");
    NEED(qkv, "vh_split_qkv_hnd_f32");
    NEED(q, "vh_split_qkv_hnd_f32");
    NEED(k, "vh_split_qkv_hnd_f32");
    NEED(v, "vh_split_qkv_hnd_f32");
    size_t per = 0, len = 0, expected = 0;
    if (mul_overflows(heads, head_dim, &per) || mul_overflows(tokens, per, &len) ||
        mul_overflows(len, 3, &expected) || qkv->len != expected || per == 0)
        return mismatch(qkv->len, expected, "vh_split_qkv_hnd_f32");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *tq = nullptr, *tk = nullptr, *tv = nullptr;
    vh_status st = new_tensor(rt->s, len, &tq, "QKV layout output allocation");
    if (!st) st = new_tensor(rt->s, len, &tk, "QKV layout output allocation");
    if (!st) st = new_tensor(rt->s, len, &tv, "QKV layout output allocation");
    if (!st)
        st = launch(s, "split_qkv_hnd", [&] {
            return vh::launch_split_qkv(s.stream, qkv->ptr, tq->ptr, tk->ptr, tv->ptr, tokens,
                                        heads, head_dim);
        });
    if (st) {
        delete tq;
        delete tk;
        delete tv;
        return st;
    }
    *q = tq;
    *k = tk;
    *v = tv;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_hnd_to_token_f32(const vh_runtime *rt, const vh_tensor *hnd,
                                         size_t tokens, size_t heads, size_t head_dim,
                                         vh_tensor **out) {
    NEED(rt, "vh_hnd_to_token_f32");
    NEED(hnd, "vh_hnd_to_token_f32");
    NEED(out, "vh_hnd_to_token_f32");
    size_t per = 0, len = 0;
    if (mul_overflows(heads, head_dim, &per) || mul_overflows(tokens, per, &len) ||
        hnd->len != len || per == 0)
        return mismatch(hnd->len, len, "vh_hnd_to_token_f32");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, len, &t, "attention layout output allocation"));
    vh_status st = launch(s, "hnd_to_token", [&] {
        return vh::launch_hnd_to_token(s.stream, hnd->ptr, t->ptr, tokens, heads, head_dim);
    });
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_token_to_chw_f32(const vh_runtime *rt, const vh_tensor *token_major,
                                         size_t tokens, size_t channels, vh_tensor **out) {
    NEED(rt, "vh_token_to_chw_f32");
    NEED(token_major, "vh_token_to_chw_f32");
    NEED(out, "vh_token_to_chw_f32");
    size_t len = 0;
    if (mul_overflows(tokens, channels, &len) || token_major->len != len || tokens == 0 ||
        channels == 0)
        return mismatch(token_major->len, len, "vh_token_to_chw_f32");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, len, &t, "CHW allocation"));
    vh_status st = launch(s, "token_to_chw", [&] {
        return vh::launch_token_to_chw(s.stream, token_major->ptr, t->ptr, tokens, channels);
    });
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_patchify_nchw_f32(const vh_runtime *rt, const vh_tensor *image,
                                          size_t height, size_t width, size_t patch,
                                          size_t channels, vh_tensor **out) {
    NEED(rt, "vh_patchify_nchw_f32");
    NEED(image, "vh_patchify_nchw_f32");
    NEED(out, "vh_patchify_nchw_f32");
    size_t hw = 0, chw = 0;
    bool bad = height == 0 || width == 0 || patch == 0 || channels == 0 ||
               height % patch != 0 || width % patch != 0 || mul_overflows(height, width, &hw) ||
               mul_overflows(hw, channels, &chw) || image->len != chw;
    if (bad)
        return fail(VH_ERR_KERNEL, "invalid NCHW patchify shape image=" + std::to_string(image->len) +
                                       ", channels=" + std::to_string(channels) +
                                       ", height=" + std::to_string(height) +
                                       ", width=" + std::to_string(width) +
                                       ", patch=" + std::to_string(patch));
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    size_t len = (height / patch) * (width / patch) * channels * patch * patch;
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, len, &t, "patchify allocation"));
    vh_status st = launch(s, "patchify_nchw", [&] {
        return vh::launch_patchify(s.stream, image->ptr, t->ptr, height, width, patch, channels);
    });
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_prepend_cls_add_pos_f32(const vh_runtime *rt, const vh_tensor *patches,
                                                const vh_tensor *cls, const vh_tensor *position,
                                                size_t patch_count, size_t embed,
                                                vh_tensor **out) {
    NEED(rt, "vh_prepend_cls_add_pos_f32");
    NEED(patches, "vh_prepend_cls_add_pos_f32");
    NEED(cls, "vh_prepend_cls_add_pos_f32");
    NEED(position, "vh_prepend_cls_add_pos_f32");
    NEED(out, "vh_prepend_cls_add_pos_f32");
    size_t plen = 0, tlen = 0;
    bool bad = embed == 0 || mul_overflows(patch_count, embed, &plen) ||
               mul_overflows(patch_count + 1, embed, &tlen) || patches->len != plen ||
               cls->len != embed || position->len != tlen;
    if (bad)
        return fail(VH_ERR_KERNEL, "invalid token assembly patches=" + std::to_string(patches->len) +
                                       ", cls=" + std::to_string(cls->len) +
                                       ", position=" + std::to_string(position->len) +
                                       ", patch_count=" + std::to_string(patch_count) +
                                       ", embed=" + std::to_string(embed));
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, tlen, &t, "token assembly allocation"));
    vh_status st = launch(s, "prepend_cls_add_pos", [&] {
        return vh::launch_prepend_cls_add_pos(s.stream, patches->ptr, cls->ptr, position->ptr,
                                              t->ptr, patch_count, embed);
    });
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

// =============================================================================
// RoPE
// =============================================================================

extern "C" vh_status vh_rope2d_f32_in_place(const vh_runtime *rt, vh_tensor *x, size_t heads,
                                            size_t n, size_t head_dim, const int64_t *pos_yx,
                                            float frequency) {
    NEED(rt, "vh_rope2d_f32_in_place");
    NEED(x, "vh_rope2d_f32_in_place");
    if (n && !pos_yx) return null_arg("vh_rope2d_f32_in_place positions");
    size_t hn = 0, expected = 0;
    if (mul_overflows(heads, n, &hn) || mul_overflows(hn, head_dim, &expected) || x->len != expected)
        return mismatch(x->len, expected, "rope2d: x size mismatch");
    if (head_dim % 4 != 0)
        return fail(VH_ERR_KERNEL, "rope2d: head_dim must be divisible by 4, got " +
                                       std::to_string(head_dim));
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    if (expected == 0) return VH_OK;
    const float *rot = nullptr;
    TRY(rope_table(s, pos_yx, n, head_dim, frequency, &rot));
    return launch(s, "rope2d", [&] { return vh::launch_rope2d(s.stream, x->ptr, heads, n, head_dim, rot); });
    GUARD_END
}

extern "C" vh_status vh_qk_norm_rope_f32_da3_base(const vh_runtime *rt, vh_tensor *q, vh_tensor *k,
                                                  const vh_tensor *q_gamma,
                                                  const vh_tensor *q_beta,
                                                  const vh_tensor *k_gamma,
                                                  const vh_tensor *k_beta,
                                                  const vh_tensor *positions_yx, size_t heads,
                                                  size_t tokens, float frequency, float epsilon) {
    NEED(rt, "vh_qk_norm_rope_f32_da3_base");
    NEED(q, "vh_qk_norm_rope_f32_da3_base");
    NEED(k, "vh_qk_norm_rope_f32_da3_base");
    NEED(q_gamma, "vh_qk_norm_rope_f32_da3_base");
    NEED(q_beta, "vh_qk_norm_rope_f32_da3_base");
    NEED(k_gamma, "vh_qk_norm_rope_f32_da3_base");
    NEED(k_beta, "vh_qk_norm_rope_f32_da3_base");
    NEED(positions_yx, "vh_qk_norm_rope_f32_da3_base");
    size_t rows = 0, expected = 0;
    bool bad = mul_overflows(heads, tokens, &rows) || mul_overflows(rows, 64, &expected) ||
               q->len != expected || k->len != expected || q_gamma->len != 64 ||
               q_beta->len != 64 || k_gamma->len != 64 || k_beta->len != 64 ||
               positions_yx->len != tokens * 2;
    if (bad) return mismatch(q->len, expected, "vh_qk_norm_rope_f32_da3_base");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    if (rows == 0) return VH_OK;
    // The positions are a device tensor here (src/cuda.rs:1184), so the
    // rotation table is built on the device from them.
    float *rot = nullptr;
    TRY(dalloc(s, tokens * 64, &rot, "RoPE table allocation"));
    vh_status st = launch(s, "rope_table", [&] {
        return vh::launch_rope_table_device(s.stream, positions_yx->ptr, tokens, frequency, rot);
    });
    if (!st)
        st = launch(s, "qk_norm_rope", [&] {
            return vh::launch_qk_norm_rope(s.stream, q->ptr, k->ptr, q_gamma->ptr, q_beta->ptr,
                                           k_gamma->ptr, k_beta->ptr, rot, rows, tokens, epsilon);
        });
    hipFreeAsync(rot, s.stream);
    return st;
    GUARD_END
}

// =============================================================================
// prepared projections
// =============================================================================

extern "C" vh_status vh_prepare_linear_f32(const vh_runtime *rt, size_t input_features,
                                           size_t output_features, const float *weight,
                                           const float *bias, const float *gamma,
                                           vh_linear **out) {
    NEED(rt, "vh_prepare_linear_f32");
    NEED(out, "vh_prepare_linear_f32");
    size_t kn = 0;
    if (mul_overflows(input_features, output_features, &kn) || (kn && !weight) ||
        (output_features && !bias))
        return fail(VH_ERR_BLAS, "linear parameter shape K=" + std::to_string(input_features) +
                                     ", N=" + std::to_string(output_features) +
                                     " does not match the provided buffers");
    if (input_features > INT32_MAX || output_features > INT32_MAX)
        return fail(VH_ERR_BLAS, "linear dimension exceeds 2^31-1");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_linear *l = new vh_linear;
    l->rt = rt->s;
    vh_status st = prepare_lin(s, input_features, output_features, weight, bias, gamma, &l->L);
    if (st) {
        delete l;
        return st;
    }
    *out = l;
    return VH_OK;
    GUARD_END
}

extern "C" void vh_linear_free(vh_linear *linear) { delete linear; }
extern "C" size_t vh_linear_input_features(const vh_linear *linear) { return linear ? linear->L.K : 0; }
extern "C" size_t vh_linear_output_features(const vh_linear *linear) { return linear ? linear->L.N : 0; }

static vh_status check_linear_input(const vh_linear *linear, const vh_tensor *input, size_t rows,
                                    const char *name) {
    NEED(linear, name);
    NEED(input, name);
    size_t expected = 0;
    if (mul_overflows(rows, linear->L.K, &expected) || input->len != expected)
        return fail(VH_ERR_BLAS, "linear input rows=" + std::to_string(rows) + ", K=" +
                                     std::to_string(linear->L.K) +
                                     " does not match device input length " +
                                     std::to_string(input->len));
    if (rows > INT32_MAX) return fail(VH_ERR_BLAS, "linear rows exceed 2^31-1");
    return VH_OK;
}

extern "C" vh_status vh_linear_run(const vh_linear *linear, const vh_tensor *input, size_t rows,
                                   vh_tensor **out) {
    TRY(check_linear_input(linear, input, rows, "vh_linear_run"));
    NEED(out, "vh_linear_run");
    GUARD_BEGIN
    RtState &s = *linear->rt;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(linear->rt, rows * linear->L.N, &t, "GEMM output allocation"));
    vh_status st = run_lin(s, linear->L, input->ptr, rows, vh::Epi::Store, t->ptr, "gemm_bias_scale");
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_linear_run_chw(const vh_linear *linear, const vh_tensor *input,
                                       size_t rows, vh_tensor **out) {
    TRY(check_linear_input(linear, input, rows, "vh_linear_run_chw"));
    NEED(out, "vh_linear_run_chw");
    GUARD_BEGIN
    RtState &s = *linear->rt;
    TRY(set_device(s));
    const size_t len = rows * linear->L.N;
    if (rows == 0 || linear->L.N == 0)
        return mismatch(len, len, "vh_linear_run_chw: token_to_chw needs tokens and channels");
    const Lin &L = linear->L;
    vh_tensor *t = nullptr;
    vh_status st = new_tensor(linear->rt, len, &t, "DPT CHW allocation");
    if (!st && !L.gamma && !L.ln_c && L.K % 32 == 0 && rows <= (size_t)INT32_MAX) {
        // The transposed product in one GEMM: the weight rows [N][K] as A and
        // the input rows as Bt, stored channel-major with the bias per
        // channel by the implicit convolution's epilogue (a 1 x 1 tap over
        // one image row of `rows` pixels); no token-major copy.
        vh::GemmArgs g{};
        g.a = L.wt;
        g.bt = input->ptr;
        g.m = L.N;
        g.n = rows;
        g.k = L.K;
        g.epi = vh::Epi::Store;
        g.c = t->ptr;
        g.bias = L.bias;
        g.conv_in_c = L.K;
        g.conv_kw = 1;
        g.conv_wp = rows;
        g.conv_ow = rows;
        st = launch(s, "gemm_bias_chw", [&] { return vh::launch_gemm(s.stream, g); });
    } else if (!st) {
        float *tmp = nullptr;
        st = dalloc(s, len, &tmp, "GEMM output allocation");
        if (!st) st = run_lin(s, L, input->ptr, rows, vh::Epi::Store, tmp, "gemm_bias_scale");
        if (!st)
            st = launch(s, "token_to_chw", [&] {
                return vh::launch_token_to_chw(s.stream, tmp, t->ptr, rows, L.N);
            });
        if (tmp) hipFreeAsync(tmp, s.stream);
    }
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_linear_run_gelu(const vh_linear *linear, const vh_tensor *input,
                                        size_t rows, vh_tensor **out) {
    TRY(check_linear_input(linear, input, rows, "vh_linear_run_gelu"));
    NEED(out, "vh_linear_run_gelu");
    if (linear->L.gamma)
        return fail(VH_ERR_BLAS, "vh_linear_run_gelu: the linear carries a LayerScale gamma");
    GUARD_BEGIN
    RtState &s = *linear->rt;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(linear->rt, rows * linear->L.N, &t, "GEMM output allocation"));
    vh_status st = run_lin(s, linear->L, input->ptr, rows, vh::Epi::Gelu, t->ptr, "gemm_bias_gelu");
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_linear_run_residual(const vh_linear *linear, const vh_tensor *input,
                                            size_t rows, vh_tensor *residual) {
    TRY(check_linear_input(linear, input, rows, "vh_linear_run_residual"));
    NEED(residual, "vh_linear_run_residual");
    if (residual->len != rows * linear->L.N)
        return mismatch(residual->len, rows * linear->L.N, "vh_linear_run_residual");
    RtState &s = *linear->rt;
    TRY(set_device(s));
    return run_lin(s, linear->L, input->ptr, rows, vh::Epi::Residual, residual->ptr,
                   "gemm_bias_scale_residual");
}

extern "C" vh_status vh_linear_run_qkv_hnd(const vh_linear *linear, const vh_tensor *input,
                                           size_t images, size_t tokens, size_t heads,
                                           const int64_t *pos_yx, float frequency, vh_tensor **q,
                                           vh_tensor **k, vh_tensor **v) {
    NEED(linear, "vh_linear_run_qkv_hnd");
    NEED(q, "vh_linear_run_qkv_hnd");
    NEED(k, "vh_linear_run_qkv_hnd");
    NEED(v, "vh_linear_run_qkv_hnd");
    size_t rows = 0;
    if (mul_overflows(images, tokens, &rows)) return mismatch(0, 0, "vh_linear_run_qkv_hnd");
    TRY(check_linear_input(linear, input, rows, "vh_linear_run_qkv_hnd"));
    if (heads == 0 || linear->L.N != heads * 3 * 64)
        return fail(VH_ERR_BLAS, "vh_linear_run_qkv_hnd: output features " +
                                     std::to_string(linear->L.N) + " != 3 * heads * 64");
    if (linear->L.gamma)
        return fail(VH_ERR_BLAS, "vh_linear_run_qkv_hnd: the QKV linear carries a gamma");
    GUARD_BEGIN
    RtState &s = *linear->rt;
    TRY(set_device(s));
    const float *rot = nullptr;
    if (pos_yx && tokens) TRY(rope_table(s, pos_yx, tokens, 64, frequency, &rot));
    const size_t len = rows * heads * 64;
    vh_tensor *tq = nullptr, *tk = nullptr, *tv = nullptr;
    vh_status st = new_tensor(linear->rt, len, &tq, "QKV output allocation");
    if (!st) st = new_tensor(linear->rt, len, &tk, "QKV output allocation");
    if (!st) st = new_tensor(linear->rt, len, &tv, "QKV output allocation");
    if (!st) st = run_qkv(s, linear->L, input->ptr, images, tokens, heads, rot, tq->ptr, tk->ptr, tv->ptr);
    if (st) {
        delete tq;
        delete tk;
        delete tv;
        return st;
    }
    *q = tq;
    *k = tk;
    *v = tv;
    return VH_OK;
    GUARD_END
}

// =============================================================================
// Q8_0
// =============================================================================

namespace {
#pragma pack(push, 1)
struct BlockQ8 {
    uint16_t d;
    int8_t qs[32];
};
#pragma pack(pop)
static_assert(sizeof(BlockQ8) == 34, "BlockQ8_0 is 34 bytes (src/lib.rs:33-38)");

vh_status new_q8(const Rt &rt, size_t rows, size_t k, vh_q8_tensor **out) {
    vh_q8_tensor *t = new vh_q8_tensor;
    t->rt = rt;
    t->rows = rows;
    t->k = k;
    vh_status st = dalloc(*rt, rows * k, &t->qs, "Q8_0 allocation");
    if (!st) st = dalloc(*rt, rows * (k / 32), &t->d, "Q8_0 allocation");
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
}

// BlockQ8_0 AoS, rows x (k/32) blocks row by row, to block-major arrays: the
// block of row r and k-slice j goes to slot j * rows + r.
void unpack_q8_aos(const void *blocks, size_t rows, size_t k, std::vector<int8_t> &qs,
                   std::vector<uint16_t> &d) {
    const size_t nbr = k / 32, nb = rows * nbr;
    qs.resize(nb * 32);
    d.resize(nb);
    const BlockQ8 *src = static_cast<const BlockQ8 *>(blocks);
    for (size_t b = 0; b < nb; b++) {
        BlockQ8 blk;
        std::memcpy(&blk, src + b, sizeof(blk));
        const size_t slot = (b % nbr) * rows + b / nbr;
        d[slot] = blk.d;
        std::memcpy(&qs[slot * 32], blk.qs, 32);
    }
}
}  // namespace

extern "C" vh_status vh_q8_0_upload(const vh_runtime *rt, const void *blocks, size_t rows,
                                    size_t k, vh_q8_tensor **out) {
    NEED(rt, "vh_q8_0_upload");
    NEED(out, "vh_q8_0_upload");
    size_t n = 0;
    if (k % 32 != 0 || mul_overflows(rows, k, &n))
        return fail(VH_ERR_KERNEL, "vh_q8_0_upload: k must be a multiple of 32, got " + std::to_string(k));
    if (n && !blocks) return null_arg("vh_q8_0_upload blocks");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    const size_t nb = n / 32;
    std::vector<int8_t> qs;
    std::vector<uint16_t> d;
    unpack_q8_aos(blocks, rows, k, qs, d);
    vh_q8_tensor *t = nullptr;
    TRY(new_q8(rt->s, rows, k, &t));
    vh_status st = h2d(s, t->qs, qs.data(), n, "Q8_0 upload");
    if (!st) st = h2d(s, t->d, d.data(), nb * 2, "Q8_0 upload");
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_q8_0_download(const vh_runtime *rt, const vh_q8_tensor *tensor,
                                      void *blocks, size_t nblocks) {
    NEED(rt, "vh_q8_0_download");
    NEED(tensor, "vh_q8_0_download");
    const size_t nb = tensor->rows * tensor->k / 32;
    if (nblocks != nb) return mismatch(nblocks, nb, "vh_q8_0_download");
    if (nb && !blocks) return null_arg("vh_q8_0_download blocks");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    std::vector<int8_t> qs(nb * 32);
    std::vector<uint16_t> d(nb);
    hipError_t e = hipSuccess;
    if (nb) {
        e = hipMemcpyAsync(qs.data(), tensor->qs, nb * 32, hipMemcpyDeviceToHost, s.stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(d.data(), tensor->d, nb * 2, hipMemcpyDeviceToHost, s.stream);
        if (e == hipSuccess) e = hipStreamSynchronize(s.stream);
    }
    if (e != hipSuccess) return fail(VH_ERR_DOWNLOAD, hip_msg("Q8_0 download", e));
    BlockQ8 *dst = static_cast<BlockQ8 *>(blocks);
    const size_t nbr = tensor->k / 32;
    for (size_t b = 0; b < nb; b++) {
        const size_t slot = (b % nbr) * tensor->rows + b / nbr;
        BlockQ8 blk;
        blk.d = d[slot];
        std::memcpy(blk.qs, &qs[slot * 32], 32);
        std::memcpy(dst + b, &blk, sizeof(blk));
    }
    return VH_OK;
    GUARD_END
}

extern "C" void vh_q8_tensor_free(vh_q8_tensor *tensor) { delete tensor; }
extern "C" size_t vh_q8_tensor_rows(const vh_q8_tensor *t) { return t ? t->rows : 0; }
extern "C" size_t vh_q8_tensor_k(const vh_q8_tensor *t) { return t ? t->k : 0; }

extern "C" vh_status vh_quantize_q8_0(const vh_runtime *rt, const vh_tensor *x, size_t rows,
                                      size_t k, vh_q8_tensor **out) {
    NEED(rt, "vh_quantize_q8_0");
    NEED(x, "vh_quantize_q8_0");
    NEED(out, "vh_quantize_q8_0");
    size_t n = 0;
    if (mul_overflows(rows, k, &n) || x->len != n)
        return mismatch(x->len, n, "x.len() must be out.len()*QK8_0");
    if (k % 32 != 0)
        return fail(VH_ERR_KERNEL, "vh_quantize_q8_0: k must be a multiple of 32, got " + std::to_string(k));
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_q8_tensor *t = nullptr;
    TRY(new_q8(rt->s, rows, k, &t));
    vh_status st = launch(s, "quantize_q8_0", [&] {
        return vh::launch_quantize_q8_0(s.stream, x->ptr, t->qs, t->d, rows, k);
    });
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_quantize_q8_0_into(const vh_runtime *rt, const vh_tensor *x, size_t rows,
                                           size_t k, vh_q8_tensor *out) {
    NEED(rt, "vh_quantize_q8_0_into");
    NEED(x, "vh_quantize_q8_0_into");
    NEED(out, "vh_quantize_q8_0_into");
    size_t n = 0;
    if (k % 32 != 0)
        return fail(VH_ERR_KERNEL, "vh_quantize_q8_0_into: k must be a multiple of 32, got " + std::to_string(k));
    if (mul_overflows(rows, k, &n) || x->len != n || out->rows != rows || out->k != k)
        return mismatch(x->len, out->rows * out->k, "x.len() must be out.len()*QK8_0");
    if (out->rt != rt->s)
        return fail(VH_ERR_KERNEL, "vh_quantize_q8_0_into: the output belongs to another runtime");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    return launch(s, "quantize_q8_0", [&] {
        return vh::launch_quantize_q8_0(s.stream, x->ptr, out->qs, out->d, rows, k);
    });
    GUARD_END
}

extern "C" vh_status vh_gemm_q8_0(const vh_runtime *rt, const vh_q8_tensor *a_q,
                                  const vh_q8_tensor *b_q, size_t m, size_t n, size_t k,
                                  vh_tensor **out) {
    NEED(rt, "vh_gemm_q8_0");
    NEED(a_q, "vh_gemm_q8_0");
    NEED(b_q, "vh_gemm_q8_0");
    NEED(out, "vh_gemm_q8_0");
    if (k % 32 != 0)
        return fail(VH_ERR_KERNEL, "k must be a multiple of QK8_0, got " + std::to_string(k));
    if (a_q->rows != m || a_q->k != k || b_q->rows != n || b_q->k != k)
        return mismatch(a_q->rows * a_q->k, m * k, "vh_gemm_q8_0 operand shape");
    if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
        return fail(VH_ERR_KERNEL, "vh_gemm_q8_0 dimension exceeds 2^31-1");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, m * n, &t, "Q8_0 GEMM output allocation"));
    vh_status st = launch(s, "gemm_q8_0", [&] {
        return vh::launch_gemm_q8_0(s.stream, a_q->qs, a_q->d, b_q->qs, b_q->d, t->ptr, m, n, k);
    });
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_gemm_q8_0_into(const vh_runtime *rt, const vh_q8_tensor *a_q,
                                       const vh_q8_tensor *b_q, size_t m, size_t n, size_t k,
                                       vh_tensor *c) {
    NEED(rt, "vh_gemm_q8_0_into");
    NEED(a_q, "vh_gemm_q8_0_into");
    NEED(b_q, "vh_gemm_q8_0_into");
    NEED(c, "vh_gemm_q8_0_into");
    if (k % 32 != 0)
        return fail(VH_ERR_KERNEL, "k must be a multiple of QK8_0, got " + std::to_string(k));
    if (a_q->rows != m || a_q->k != k || b_q->rows != n || b_q->k != k)
        return mismatch(a_q->rows * a_q->k, m * k, "vh_gemm_q8_0_into operand shape");
    size_t mn = 0;
    if (mul_overflows(m, n, &mn) || c->len != mn) return mismatch(c->len, mn, "c.len() must be m * n");
    if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
        return fail(VH_ERR_KERNEL, "vh_gemm_q8_0_into dimension exceeds 2^31-1");
    if (c->rt != rt->s || a_q->rt != rt->s || b_q->rt != rt->s)
        return fail(VH_ERR_KERNEL, "vh_gemm_q8_0_into: a tensor belongs to another runtime");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    return launch(s, "gemm_q8_0", [&] {
        return vh::launch_gemm_q8_0(s.stream, a_q->qs, a_q->d, b_q->qs, b_q->d, c->ptr, m, n, k);
    });
    GUARD_END
}

// ---- Q8_0 projection --------------------------------------------------------

extern "C" vh_status vh_prepare_linear_q8_0(const vh_runtime *rt, size_t input_features,
                                            size_t output_features, const void *weight_blocks,
                                            const float *bias, const float *gamma,
                                            vh_linear_q8 **out) {
    NEED(rt, "vh_prepare_linear_q8_0");
    NEED(out, "vh_prepare_linear_q8_0");
    size_t kn = 0;
    if (input_features % 32 != 0)
        return fail(VH_ERR_KERNEL, "vh_prepare_linear_q8_0: input_features must be a multiple of "
                                   "QK8_0, got " + std::to_string(input_features));
    if (mul_overflows(input_features, output_features, &kn) || (kn && !weight_blocks))
        return fail(VH_ERR_BLAS, "linear parameter shape K=" + std::to_string(input_features) +
                                     ", N=" + std::to_string(output_features) +
                                     " does not match the provided buffers");
    if (input_features > INT32_MAX || output_features > INT32_MAX)
        return fail(VH_ERR_BLAS, "linear dimension exceeds 2^31-1");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    std::vector<int8_t> qs;
    std::vector<uint16_t> d;
    unpack_q8_aos(weight_blocks, output_features, input_features, qs, d);
    vh_linear_q8 *l = new vh_linear_q8;
    l->rt = rt->s;
    Q8Lin &L = l->L;
    vh_status st = dalloc(s, kn, &L.qs, "Q8_0 weight allocation");
    if (!st) st = dalloc(s, kn / 32, &L.d, "Q8_0 weight allocation");
    if (!st) st = h2d(s, L.qs, qs.data(), kn, "Q8_0 weight upload");
    if (!st) st = h2d(s, L.d, d.data(), kn / 32 * sizeof(uint16_t), "Q8_0 weight upload");
    if (!st && bias) st = upload_array(s, bias, output_features, &L.bias, "linear bias upload");
    if (!st && gamma) st = upload_array(s, gamma, output_features, &L.gamma, "linear gamma upload");
    if (st) {
        delete l;
        return st;
    }
    L.K = input_features;
    L.N = output_features;
    *out = l;
    return VH_OK;
    GUARD_END
}

extern "C" void vh_linear_q8_0_free(vh_linear_q8 *linear) { delete linear; }
extern "C" size_t vh_linear_q8_0_input_features(const vh_linear_q8 *linear) {
    return linear ? linear->L.K : 0;
}
extern "C" size_t vh_linear_q8_0_output_features(const vh_linear_q8 *linear) {
    return linear ? linear->L.N : 0;
}

static vh_status check_q8_input(const vh_linear_q8 *linear, const vh_tensor *input, size_t rows,
                                const char *name) {
    NEED(linear, name);
    NEED(input, name);
    size_t expected = 0;
    if (mul_overflows(rows, linear->L.K, &expected) || input->len != expected)
        return fail(VH_ERR_BLAS, "linear input rows=" + std::to_string(rows) + ", K=" +
                                     std::to_string(linear->L.K) +
                                     " does not match device input length " +
                                     std::to_string(input->len));
    if (rows > INT32_MAX) return fail(VH_ERR_BLAS, "linear rows exceed 2^31-1");
    return VH_OK;
}

static vh_status q8_linear_new(const vh_linear_q8 *linear, const vh_tensor *input, size_t rows,
                               vh::Epi epi, const char *name, vh_tensor **out) {
    TRY(check_q8_input(linear, input, rows, name));
    NEED(out, name);
    if (epi == vh::Epi::Gelu && linear->L.gamma)
        return fail(VH_ERR_BLAS, std::string(name) + ": the linear carries a LayerScale gamma");
    GUARD_BEGIN
    RtState &s = *linear->rt;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(linear->rt, rows * linear->L.N, &t, "GEMM output allocation"));
    vh_status st = rows ? run_q8(s, linear->L, input->ptr, rows, epi, t->ptr, name) : VH_OK;
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_linear_q8_0_run(const vh_linear_q8 *linear, const vh_tensor *input,
                                        size_t rows, vh_tensor **out) {
    return q8_linear_new(linear, input, rows, vh::Epi::Store, "gemm_q8_0_bias_scale", out);
}

extern "C" vh_status vh_linear_q8_0_run_gelu(const vh_linear_q8 *linear, const vh_tensor *input,
                                             size_t rows, vh_tensor **out) {
    return q8_linear_new(linear, input, rows, vh::Epi::Gelu, "gemm_q8_0_bias_gelu", out);
}

extern "C" vh_status vh_linear_q8_0_run_residual(const vh_linear_q8 *linear,
                                                 const vh_tensor *input, size_t rows,
                                                 vh_tensor *residual) {
    TRY(check_q8_input(linear, input, rows, "vh_linear_q8_0_run_residual"));
    NEED(residual, "vh_linear_q8_0_run_residual");
    if (residual->len != rows * linear->L.N)
        return mismatch(residual->len, rows * linear->L.N, "vh_linear_q8_0_run_residual");
    GUARD_BEGIN
    RtState &s = *linear->rt;
    TRY(set_device(s));
    if (rows == 0) return VH_OK;
    return run_q8(s, linear->L, input->ptr, rows, vh::Epi::Residual, residual->ptr,
                  "gemm_q8_0_bias_scale_residual");
    GUARD_END
}

// =============================================================================
// DA3-BASE encoder block
// =============================================================================

namespace {
constexpr size_t kDim = 768, kHeads = 12, kMlp = 3072;

vh_status upload_small(RtState &s, const float *h, size_t n, float **out, const char *what) {
    if (!h) return null_arg(what);
    return upload_array(s, h, n, out, what);
}

// One pre-norm block, in place on x.  x_chunks (encoder runs): on entry,
// the chunks per row of x's row statistics in the block workspace (the
// previous f32 block's fc2 wrote them; 0: none); on return, those this
// block's fc2 wrote.
vh_status block_run(RtState &s, const vh_block &b, float *x, size_t images, size_t tokens,
                    const int64_t *pos, float freq, float eps, int *x_chunks = nullptr) {
    const size_t M = images * tokens;
    const size_t D = kDim;
    float *ws = nullptr;
    TRY(workspace(s, M * (4 * D + kMlp + 2 * (D / 16)), &ws));
    float *q = ws, *k = q + M * D, *v = k + M * D, *att = v + M * D, *f = att + M * D;
    float *rs = f + M * kMlp;  // row statistics [M][chunks <= D / 16][mean, M2]
    const int in_chunks = x_chunks ? *x_chunks : 0;
    if (x_chunks) *x_chunks = 0;
    const float *rot = nullptr;
    if (pos) {
        TRY(rope_table(s, pos, tokens, 64, freq, &rot));
    } else if (b.qn_g) {
        // A late block without positions: every token at (0, 0), whose
        // rotation (sin 0, cos 1) leaves the normalised rows unchanged.
        std::vector<int64_t> zero(tokens * 2, 0);
        TRY(rope_table(s, zero.data(), tokens, 64, freq, &rot));
    }
    if (b.q8) {
        // Q8_0 projections: each GEMM takes Q8_0 rows, so the LayerNorms
        // write Q8_0 directly.
        const RowNorm ln1{b.ln1_g, b.ln1_b, nullptr, eps};
        const float *qin = x;
        const RowNorm *n1 = &ln1;
        if (b.qn_g) {
            TRY(run_q8_qkv(s, b.qqkv, qin, images, tokens, nullptr, q, k, v, n1));
            TRY(launch(s, "qk_norm_rope", [&] {
                return vh::launch_qk_norm_rope(s.stream, q, k, b.qn_g, b.qn_b, b.kn_g, b.kn_b,
                                               rot, M * kHeads, tokens, eps);
            }));
        } else {
            TRY(run_q8_qkv(s, b.qqkv, qin, images, tokens, rot, q, k, v, n1));
        }
        // The attention merge writes Q8_0 rows directly when the keys are
        // split; otherwise the f32 output is quantised.
        Q8Rows a;
        TRY(q8_workspace(s, M, D, &a.qs, &a.d));
        bool quantized = false;
        TRY(flash(s, q, k, v, att, images * kHeads, tokens, kHeads, true, a.qs, a.d, &quantized));
        if (!quantized)
            TRY(launch(s, "quantize_q8_0", [&] {
                return vh::launch_quantize_q8_0(s.stream, att, a.qs, a.d, M, D);
            }));
        TRY(launch(s, "gemm_q8_0_proj_residual", [&] {
            return vh::launch_gemm_q8_0(s.stream, a.qs, a.d, b.qproj.qs, b.qproj.d, x, M, D, D,
                                        vh::Epi::Residual, b.qproj.bias, b.qproj.gamma);
        }));
        // fc1 quantises its GELU output for fc2 in its epilogue when its
        // tile allows (the f32 output is quantised otherwise).  Its input
        // rows and its output rows need separate Q8_0 buffers: the output
        // goes to the block workspace, past the f32 rows of f.
        const RowNorm ln2{b.ln2_g, b.ln2_b, nullptr, eps};
        Q8Rows hin;
        TRY(q8_rows(s, x, M, D, &ln2, &hin));
        int8_t *fq = reinterpret_cast<int8_t *>(f);  // M x kMlp bytes of values ...
        uint16_t *fd = reinterpret_cast<uint16_t *>(fq + M * kMlp);  // ... then the scales
        bool fq_ready = false;
        TRY(launch(s, "gemm_q8_0_fc1_gelu", [&] {
            return vh::launch_gemm_q8_0(s.stream, hin.qs, hin.d, b.qfc1.qs, b.qfc1.d, f, M, kMlp,
                                        D, vh::Epi::Gelu, b.qfc1.bias, nullptr, fq, fd, &fq_ready);
        }));
        if (!fq_ready) return run_q8(s, b.qfc2, f, M, vh::Epi::Residual, x, "gemm_q8_0_fc2_residual");
        return launch(s, "gemm_q8_0_fc2_residual", [&] {
            return vh::launch_gemm_q8_0(s.stream, fq, fd, b.qfc2.qs, b.qfc2.d, x, M, D, kMlp,
                                        vh::Epi::Residual, b.qfc2.bias, b.qfc2.gamma);
        });
    }
    // f32 projections: LayerNorm 1 and 2 are folded into the QKV and fc1
    // GEMMs (prepare_lin_ln), which read the residual stream x itself and
    // take its row statistics from the Residual GEMM before them when that
    // one wrote them (the out-projection for fc1, the previous block's fc2
    // for QKV), else from their own A slices.
    const float *qkv_stats = in_chunks ? rs : nullptr;
    if (b.qn_g) {
        // Late block: QKV with bias only, then LayerNorm of every 64-wide Q
        // and K head row fused with the RoPE (src/specialized.rs:278-316).
        TRY(run_qkv(s, b.qkv, x, images, tokens, kHeads, nullptr, q, k, v, eps, qkv_stats, in_chunks));
        TRY(launch(s, "qk_norm_rope", [&] {
            return vh::launch_qk_norm_rope(s.stream, q, k, b.qn_g, b.qn_b, b.kn_g, b.kn_b, rot,
                                           M * kHeads, tokens, eps);
        }));
    } else {
        TRY(run_qkv(s, b.qkv, x, images, tokens, kHeads, rot, q, k, v, eps, qkv_stats, in_chunks));
    }
    TRY(flash(s, q, k, v, att, images * kHeads, tokens, kHeads, true));
    int proj_chunks = 0;
    TRY(run_lin(s, b.proj, att, M, vh::Epi::Residual, x, "gemm_proj_residual", nullptr, 0.0f,
                ChunkStats{nullptr, 0, rs, &proj_chunks}));
    TRY(run_lin(s, b.fc1, x, M, vh::Epi::Gelu, f, "gemm_fc1_gelu", nullptr, eps,
                ChunkStats{proj_chunks ? rs : nullptr, (size_t)proj_chunks, nullptr, nullptr}));
    if (!x_chunks) return run_lin(s, b.fc2, f, M, vh::Epi::Residual, x, "gemm_fc2_residual");
    return run_lin(s, b.fc2, f, M, vh::Epi::Residual, x, "gemm_fc2_residual", nullptr, 0.0f,
                   ChunkStats{nullptr, 0, rs, x_chunks});
}

vh_status check_block_x(const vh_tensor *x, size_t images, size_t tokens) {
    size_t m = 0, len = 0;
    if (mul_overflows(images, tokens, &m) || mul_overflows(m, kDim, &len) || x->len != len)
        return mismatch(x->len, len, "DA3 block input");
    if (m > INT32_MAX / 4 || images * kHeads > 65535)
        return fail(VH_ERR_KERNEL, "DA3 block shape exceeds the launch grid");
    return VH_OK;
}
}  // namespace

static vh_status block_prepare(const vh_runtime *rt, const vh_block_params *p, bool q8,
                               vh_block **out) {
    NEED(rt, "vh_block_prepare");
    NEED(p, "vh_block_prepare");
    NEED(out, "vh_block_prepare");
    const float *req[] = {p->ln1_gamma, p->ln1_beta, p->w_qkv, p->b_qkv, p->w_proj,
                          p->b_proj,    p->ls1,      p->ln2_gamma, p->ln2_beta, p->w_fc1,
                          p->b_fc1,     p->w_fc2,    p->b_fc2, p->ls2};
    for (const float *r : req)
        if (!r) return null_arg("vh_block_prepare parameter");
    const int qk_norm = !!p->q_norm_gamma + !!p->q_norm_beta + !!p->k_norm_gamma + !!p->k_norm_beta;
    if (qk_norm != 0 && qk_norm != 4)
        return fail(VH_ERR_INVALID_ARGUMENT,
                    "vh_block_prepare: give all four Q/K LayerNorm vectors or none");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_block *b = new vh_block;
    b->rt = rt->s;
    b->q8 = q8;
    vh_status st;
    if (q8) {
        st = prepare_q8_from_f32(s, kDim, 3 * kDim, p->w_qkv, p->b_qkv, nullptr, &b->qqkv);
        if (!st) st = prepare_q8_from_f32(s, kDim, kDim, p->w_proj, p->b_proj, p->ls1, &b->qproj);
        if (!st) st = prepare_q8_from_f32(s, kDim, kMlp, p->w_fc1, p->b_fc1, nullptr, &b->qfc1);
        if (!st) st = prepare_q8_from_f32(s, kMlp, kDim, p->w_fc2, p->b_fc2, p->ls2, &b->qfc2);
    } else {
        st = prepare_lin_ln(s, kDim, 3 * kDim, p->w_qkv, p->b_qkv, p->ln1_gamma, p->ln1_beta, &b->qkv);
        if (!st) st = prepare_lin(s, kDim, kDim, p->w_proj, p->b_proj, p->ls1, &b->proj);
        if (!st) st = prepare_lin_ln(s, kDim, kMlp, p->w_fc1, p->b_fc1, p->ln2_gamma, p->ln2_beta, &b->fc1);
        if (!st) st = prepare_lin(s, kMlp, kDim, p->w_fc2, p->b_fc2, p->ls2, &b->fc2);
    }
    if (!st) st = upload_small(s, p->ln1_gamma, kDim, &b->ln1_g, "ln1 gamma");
    if (!st) st = upload_small(s, p->ln1_beta, kDim, &b->ln1_b, "ln1 beta");
    if (!st) st = upload_small(s, p->ln2_gamma, kDim, &b->ln2_g, "ln2 gamma");
    if (!st) st = upload_small(s, p->ln2_beta, kDim, &b->ln2_b, "ln2 beta");
    if (qk_norm) {
        if (!st) st = upload_small(s, p->q_norm_gamma, 64, &b->qn_g, "q norm gamma");
        if (!st) st = upload_small(s, p->q_norm_beta, 64, &b->qn_b, "q norm beta");
        if (!st) st = upload_small(s, p->k_norm_gamma, 64, &b->kn_g, "k norm gamma");
        if (!st) st = upload_small(s, p->k_norm_beta, 64, &b->kn_b, "k norm beta");
    }
    if (st) {
        delete b;
        return st;
    }
    *out = b;
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_block_prepare(const vh_runtime *rt, const vh_block_params *p,
                                      vh_block **out) {
    return block_prepare(rt, p, false, out);
}

extern "C" vh_status vh_block_prepare_q8_0(const vh_runtime *rt, const vh_block_params *p,
                                           vh_block **out) {
    return block_prepare(rt, p, true, out);
}

extern "C" int vh_block_is_q8_0(const vh_block *block) { return block && block->q8; }

extern "C" void vh_block_free(vh_block *block) { delete block; }

extern "C" vh_status vh_vit_block_run(const vh_runtime *rt, const vh_block *block, vh_tensor *x,
                                      size_t images, size_t tokens, const int64_t *pos_yx,
                                      float rope_frequency, float epsilon) {
    NEED(rt, "vh_vit_block_run");
    NEED(block, "vh_vit_block_run");
    NEED(x, "vh_vit_block_run");
    TRY(check_block_x(x, images, tokens));
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    if (images * tokens == 0) return VH_OK;
    return block_run(s, *block, x->ptr, images, tokens, pos_yx, rope_frequency, epsilon);
    GUARD_END
}

extern "C" vh_status vh_encoder_run(const vh_runtime *rt, const vh_block *const *blocks,
                                    size_t layers, vh_tensor *x, size_t images, size_t tokens,
                                    const int64_t *pos_yx, float rope_frequency, float epsilon) {
    NEED(rt, "vh_encoder_run");
    NEED(x, "vh_encoder_run");
    if (layers && !blocks) return null_arg("vh_encoder_run blocks");
    for (size_t i = 0; i < layers; i++)
        if (!blocks[i]) return null_arg("vh_encoder_run block");
    TRY(check_block_x(x, images, tokens));
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    if (images * tokens == 0) return VH_OK;
    // Each f32 block's fc2 leaves the row statistics of its output for the
    // next block's QKV (a Q8_0 block normalises its own input).
    int x_chunks = 0;
    for (size_t i = 0; i < layers; i++) {
        if (blocks[i]->q8) x_chunks = 0;
        TRY(block_run(s, *blocks[i], x->ptr, images, tokens, pos_yx, rope_frequency, epsilon,
                      blocks[i]->q8 ? nullptr : &x_chunks));
    }
    return VH_OK;
    GUARD_END
}

// =============================================================================
// DPT head: convolution, transposed convolution, bilinear resize
// =============================================================================

struct vh_conv2d {
    Rt rt;
    size_t in_c = 0, out_c = 0, kh = 0, kw = 0, stride = 0, pad = 0;
    // in_c % 4 == 0: weight [out_c][kh][kw][in_c] and channel-last patches;
    // else OIHW = [out_c][in_c*kh*kw].  Either is the GEMM's Bt operand.
    bool hwc = false;
    float *w = nullptr;
    float *bias = nullptr;  // [out_c] or null
    ~vh_conv2d() {
        if (!rt) return;
        hipSetDevice(rt->device);
        for (float *p : {w, bias})
            if (p) hipFreeAsync(p, rt->stream);
    }
};

struct vh_conv_transpose2d {
    Rt rt;
    size_t in_c = 0, out_c = 0, kh = 0, kw = 0, stride = 0;
    bool nonoverlap = false;  // kernel == stride: one GEMM plus a patch scatter
    float *w = nullptr;       // nonoverlap: [out_c*kh*kw][in_c]; else IOHW as given
    float *bias = nullptr;    // [out_c] or null
    float *bias_x = nullptr;  // nonoverlap: bias repeated per (ky, kx), [out_c*kh*kw]
    ~vh_conv_transpose2d() {
        if (!rt) return;
        hipSetDevice(rt->device);
        for (float *p : {w, bias, bias_x})
            if (p) hipFreeAsync(p, rt->stream);
    }
};

namespace {

vh_status check_tensor_len(const vh_tensor *t, size_t expected, const char *what) {
    if (t->len != expected) return mismatch(t->len, expected, what);
    return VH_OK;
}

// c [rows][cols] = a [rows][k] . bt [cols][k]^T (+ bias[col]), the fp32-MFMA GEMM.
vh_status gemm_nt(RtState &s, const float *a, const float *bt, const float *bias, float *c,
                  size_t rows, size_t cols, size_t k, const char *name) {
    vh::GemmArgs g{};
    g.a = a;
    g.bt = bt;
    g.m = rows;
    g.n = cols;
    g.k = k;
    g.epi = vh::Epi::Store;
    g.c = c;
    g.bias = bias;
    TRY(splitk_workspace(s, rows, cols, &g.ws, &g.ws_floats));
    TRY(tail_workspace(s, g));
    return launch(s, name, [&] { return vh::launch_gemm(s.stream, g); });
}

// Convolution of a CHW input in place of conv2d (src/conv.rs:877-945): the
// patches as colT [pixels][K], one GEMM against the OIHW weight with the
// bias in its epilogue, then [pixels][out_c] -> CHW.
vh_status conv_run(RtState &s, const vh_conv2d &c, const float *in, size_t ih, size_t iw,
                   bool relu, float *out) {
    const size_t oh = (ih + 2 * c.pad - c.kh) / c.stride + 1;
    const size_t ow = (iw + 2 * c.pad - c.kw) / c.stride + 1;
    const size_t npix = oh * ow, K = c.in_c * c.kh * c.kw;
    const bool plain = c.kh == 1 && c.kw == 1 && c.stride == 1 && c.pad == 0 && !relu;
    float *xh = nullptr, *col = nullptr, *tmp = nullptr;
    vh_status st = VH_OK;
    // The direct form reads the image with eight 4-byte loads per thread and
    // k-slice where the staged GEMM issues two 16-byte ones, but saves the
    // staging launches and copies, and its balanced tail splits the K of
    // grids too small to fill the GPU.  Measured on MI355X (3x3, per call,
    // direct against staged): 128 -> 128 on 96 x 144 48.6 vs 74.9 us, 768 ->
    // 128 on 12 x 18 48.4 vs 235.7, 384 -> 128 on 24 x 36 27.9 vs 124.3,
    // 768 -> 768 stride 2 on 24 x 36 57.4 vs 82.8, 64 -> 32 on 384 x 576
    // 169.2 vs 173.3; only stride-1 convolutions with K >= 1152 and more than
    // 4 M outputs stay staged (128 -> 128 on 192 x 288: 168.7 vs 160.4).
    // VESTRA_HIP_CONV_DIRECT=0|1 forces either form (A/B runs).
    const char *direct_env = std::getenv("VESTRA_HIP_CONV_DIRECT");
    const bool direct_default =
        !(c.stride == 1 && K >= 1152 && npix * c.out_c > ((size_t)4 << 20));
    const bool direct_ok = direct_env ? std::atoi(direct_env) != 0 : direct_default;
    if (direct_ok && c.hwc && c.in_c % 32 == 0) {
        // Direct implicit GEMM: the GEMM reads the CHW image in place (taps
        // outside the image as zeros, ReLU applied on load) and stores the
        // CHW output from its epilogue; no staging copies.
        vh::GemmArgs g{};
        g.a = c.w;
        g.bt = in;
        g.m = c.out_c;
        g.n = npix;
        g.k = K;
        g.epi = vh::Epi::Store;
        g.c = out;
        g.bias = c.bias;
        g.conv_in_c = c.in_c;
        g.conv_kw = c.kw;
        g.conv_ow = ow;
        g.conv_ih = ih;
        g.conv_iw = iw;
        g.conv_stride = c.stride;
        g.conv_pad = c.pad;
        g.conv_relu = relu;
        TRY(tail_workspace(s, g));
        return launch(s, "conv_gemm", [&] { return vh::launch_gemm(s.stream, g); });
    }
    if (c.hwc && c.stride == 1 && c.in_c % 32 == 0 && !plain) {
        // Implicit GEMM: the GEMM reads each tap's rows straight from the
        // zero-padded channel-last image, computes the outputs on the padded
        // grid (wp - ow junk columns per row) with the output channels as
        // rows, and stores the CHW output directly, junk columns dropped.
        const size_t wp = iw + 2 * c.pad, hp = ih + 2 * c.pad;
        const size_t rows = hp * wp + c.kw - 1;
        st = dalloc(s, rows * c.in_c, &xh, "convolution staging allocation");
        if (!st)
            st = launch(s, "conv_to_padded_hwc", [&] {
                return vh::launch_chw_to_padded_hwc(s.stream, in, xh, c.in_c, ih, iw, c.pad, rows,
                                                    relu);
            });
        if (!st) {
            vh::GemmArgs g{};
            g.a = c.w;
            g.bt = xh;
            g.m = c.out_c;
            g.n = oh * wp;
            g.k = K;
            g.epi = vh::Epi::Store;
            g.c = out;
            g.bias = c.bias;
            g.conv_in_c = c.in_c;
            g.conv_kw = c.kw;
            g.conv_wp = wp;
            g.conv_ow = ow;
            st = launch(s, "conv_gemm", [&] { return vh::launch_gemm(s.stream, g); });
        }
        if (xh) hipFreeAsync(xh, s.stream);
        return st;
    }
    if (c.hwc && !plain) {
        // Channel-last copy of the input, then one contiguous run per tap.
        st = dalloc(s, ih * iw * c.in_c, &xh, "convolution staging allocation");
        if (!st)
            st = launch(s, "conv_to_hwc", [&] {
                return vh::launch_transpose(s.stream, in, xh, c.in_c, ih * iw);
            });
    }
    if (!st) st = dalloc(s, npix * K, &col, "convolution patch allocation");
    if (!st) st = dalloc(s, npix * c.out_c, &tmp, "convolution output allocation");
    if (!st) {
        st = launch(s, plain ? "conv_to_hwc" : "im2col", [&] {
            if (plain) return vh::launch_transpose(s.stream, in, col, c.in_c, npix);
            if (c.hwc)
                return vh::launch_im2col_hwc(s.stream, xh, col, c.in_c, ih, iw, c.kh, c.kw,
                                             c.stride, c.pad, oh, ow, relu);
            return vh::launch_im2col_t(s.stream, in, col, c.in_c, ih, iw, c.kh, c.kw, c.stride,
                                       c.pad, oh, ow, relu);
        });
    }
    if (!st) st = gemm_nt(s, col, c.w, c.bias, tmp, npix, c.out_c, K, "conv_gemm");
    if (!st)
        st = launch(s, "conv_to_chw", [&] {
            return vh::launch_transpose(s.stream, tmp, out, npix, c.out_c);
        });
    for (float *p : {xh, col, tmp})
        if (p) hipFreeAsync(p, s.stream);
    return st;
}

vh_status conv_geometry(const vh_conv2d *c, const vh_tensor *input, size_t ih, size_t iw,
                        size_t *oh, size_t *ow) {
    size_t plane = 0, len = 0;
    if (mul_overflows(ih, iw, &plane) || mul_overflows(plane, c->in_c, &len))
        return fail(VH_ERR_KERNEL, "conv2d: input size overflows");
    TRY(check_tensor_len(input, len, "conv2d input"));
    if (ih + 2 * c->pad < c->kh || iw + 2 * c->pad < c->kw)
        return fail(VH_ERR_KERNEL, "conv2d: kernel larger than the padded input");
    *oh = (ih + 2 * c->pad - c->kh) / c->stride + 1;
    *ow = (iw + 2 * c->pad - c->kw) / c->stride + 1;
    size_t npix = *oh * *ow, cells = 0, outs = 0;
    if (mul_overflows(npix, c->in_c * c->kh * c->kw, &cells) || cells > (size_t)INT32_MAX ||
        mul_overflows(npix, c->out_c, &outs) || outs > (size_t)INT32_MAX ||
        npix > (size_t)INT32_MAX / 2 || ih > INT32_MAX / 2 || iw > INT32_MAX / 2 ||
        (npix + 31) / 32 > 65535 || *oh > 65535)
        return fail(VH_ERR_KERNEL, "conv2d: shape exceeds the supported size");
    return VH_OK;
}

vh_status prepare_conv(const vh_runtime *rt, size_t in_c, size_t out_c, size_t kh, size_t kw,
                       size_t stride, size_t pad, const float *weight, const float *bias,
                       vh_conv2d **out) {
    NEED(rt, "vh_prepare_conv2d_f32");
    NEED(out, "vh_prepare_conv2d_f32");
    if (!in_c || !out_c || !kh || !kw || !stride)
        return fail(VH_ERR_KERNEL, "conv2d: channels, kernel and stride must be non-zero");
    size_t n = 0;
    if (mul_overflows(out_c, in_c * kh * kw, &n) || in_c > INT32_MAX / (kh * kw) ||
        out_c > INT32_MAX)
        return fail(VH_ERR_KERNEL, "conv2d: weight size overflows");
    NEED(weight, "vh_prepare_conv2d_f32 weight");
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_conv2d *c = new vh_conv2d;
    c->rt = rt->s;
    c->in_c = in_c;
    c->out_c = out_c;
    c->kh = kh;
    c->kw = kw;
    c->stride = stride;
    c->pad = pad;
    c->hwc = in_c % 4 == 0;
    vh_status st;
    if (c->hwc) {
        // OIHW -> [out_c][kh][kw][in_c], the k order of the channel-last patches.
        std::vector<float> packed(n);
        const size_t taps = kh * kw;
        for (size_t o = 0; o < out_c; o++)
            for (size_t i = 0; i < in_c; i++)
                for (size_t t = 0; t < taps; t++)
                    packed[(o * taps + t) * in_c + i] = weight[(o * in_c + i) * taps + t];
        st = upload_array(s, packed.data(), n, &c->w, "conv2d weight upload");
    } else {
        st = upload_array(s, weight, n, &c->w, "conv2d weight upload");
    }
    if (!st && bias) st = upload_array(s, bias, out_c, &c->bias, "conv2d bias upload");
    if (st) {
        delete c;
        return st;
    }
    *out = c;
    return VH_OK;
}

vh_status conv_new(const vh_conv2d *conv, const vh_tensor *input, size_t ih, size_t iw,
                   bool relu, vh_tensor **out, const char *name) {
    NEED(conv, name);
    NEED(input, name);
    NEED(out, name);
    size_t oh = 0, ow = 0;
    TRY(conv_geometry(conv, input, ih, iw, &oh, &ow));
    RtState &s = *conv->rt;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(conv->rt, conv->out_c * oh * ow, &t, "conv2d output allocation"));
    vh_status st = conv_run(s, *conv, input->ptr, ih, iw, relu, t->ptr);
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
}

vh_status prepare_conv_t(const vh_runtime *rt, size_t in_c, size_t out_c, size_t kh, size_t kw,
                         size_t stride, const float *weight, const float *bias,
                         vh_conv_transpose2d **out) {
    NEED(rt, "vh_prepare_conv_transpose2d_f32");
    NEED(out, "vh_prepare_conv_transpose2d_f32");
    if (!in_c || !out_c || !kh || !kw || !stride)
        return fail(VH_ERR_KERNEL, "conv_transpose2d: channels, kernel and stride must be non-zero");
    size_t n = 0;
    if (mul_overflows(in_c, out_c * kh * kw, &n) || out_c * kh * kw > INT32_MAX ||
        in_c > INT32_MAX)
        return fail(VH_ERR_KERNEL, "conv_transpose2d: weight size overflows");
    NEED(weight, "vh_prepare_conv_transpose2d_f32 weight");
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_conv_transpose2d *c = new vh_conv_transpose2d;
    c->rt = rt->s;
    c->in_c = in_c;
    c->out_c = out_c;
    c->kh = kh;
    c->kw = kw;
    c->stride = stride;
    c->nonoverlap = kh == stride && kw == stride;
    vh_status st = VH_OK;
    if (c->nonoverlap) {
        // prepare_nonoverlap_transpose_f32 (src/specialized.rs:148-174): IOHW
        // -> [out_c][kh][kw][in_c], the GEMM's Bt operand.
        std::vector<float> packed(n);
        const size_t taps = kh * kw;
        for (size_t o = 0; o < out_c; o++)
            for (size_t t = 0; t < taps; t++)
                for (size_t i = 0; i < in_c; i++)
                    packed[(o * taps + t) * in_c + i] = weight[(i * out_c + o) * taps + t];
        st = upload_array(s, packed.data(), n, &c->w, "conv_transpose2d weight upload");
        if (!st && bias) {
            std::vector<float> bx(out_c * taps);
            for (size_t o = 0; o < out_c; o++)
                for (size_t t = 0; t < taps; t++) bx[o * taps + t] = bias[o];
            st = upload_array(s, bx.data(), bx.size(), &c->bias_x, "conv_transpose2d bias upload");
        }
    } else {
        st = upload_array(s, weight, n, &c->w, "conv_transpose2d weight upload");
        if (!st && bias) st = upload_array(s, bias, out_c, &c->bias, "conv_transpose2d bias upload");
    }
    if (st) {
        delete c;
        return st;
    }
    *out = c;
    return VH_OK;
}

vh_status conv_t_new(const vh_conv_transpose2d *c, const vh_tensor *input, size_t ih, size_t iw,
                     vh_tensor **out) {
    NEED(c, "vh_conv_transpose2d_run");
    NEED(input, "vh_conv_transpose2d_run");
    NEED(out, "vh_conv_transpose2d_run");
    size_t plane = 0, len = 0;
    if (mul_overflows(ih, iw, &plane) || mul_overflows(plane, c->in_c, &len))
        return fail(VH_ERR_KERNEL, "conv_transpose2d: input size overflows");
    TRY(check_tensor_len(input, len, "conv_transpose2d input"));
    if (ih == 0 || iw == 0)
        return fail(VH_ERR_KERNEL, "conv_transpose2d: empty input (the output size needs ih, iw >= 1)");
    const size_t oh = (ih - 1) * c->stride + c->kh, ow = (iw - 1) * c->stride + c->kw;
    size_t olen = 0;
    if (mul_overflows(oh, ow, &olen) || mul_overflows(olen, c->out_c, &olen) ||
        olen > (size_t)INT32_MAX * 4 || oh > INT32_MAX / 2 || ow > INT32_MAX / 2 ||
        (plane + 31) / 32 > 65535)
        return fail(VH_ERR_KERNEL, "conv_transpose2d: shape exceeds the supported size");
    GUARD_BEGIN
    RtState &s = *c->rt;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(c->rt, olen, &t, "conv_transpose2d output allocation"));
    vh_status st = VH_OK;
    if (c->nonoverlap && c->in_c % 32 == 0) {
        // One GEMM with the weight rows (oc, ky, kx) as the tile rows and the
        // input pixels as its columns, read from the CHW input in place,
        // stored straight to CHW by its patch-scatter epilogue.
        // VESTRA_HIP_CONV_DIRECT=0 reads a channel-last copy instead (A/B
        // runs; the same products in the same order, so the same bits).
        const char *direct_env = std::getenv("VESTRA_HIP_CONV_DIRECT");
        const bool direct = !(direct_env && direct_env[0] == '0');
        float *xt = nullptr;
        if (!direct) {
            st = dalloc(s, plane * c->in_c, &xt, "conv_transpose2d staging allocation");
            if (!st)
                st = launch(s, "conv_transpose_to_hwc", [&] {
                    return vh::launch_transpose(s.stream, input->ptr, xt, c->in_c, plane);
                });
        }
        if (!st) {
            vh::GemmArgs g{};
            g.a = c->w;
            g.bt = direct ? input->ptr : xt;
            g.scatter_chw = direct;
            g.m = c->out_c * c->kh * c->kw;
            g.n = plane;
            g.k = c->in_c;
            g.epi = vh::Epi::Store;
            g.c = t->ptr;
            g.bias = c->bias_x;
            g.scatter_kh = c->kh;
            g.scatter_kw = c->kw;
            g.scatter_iw = iw;
            st = launch(s, "conv_transpose_gemm", [&] { return vh::launch_gemm(s.stream, g); });
        }
        if (xt) hipFreeAsync(xt, s.stream);
    } else if (c->nonoverlap) {
        const size_t cols = c->out_c * c->kh * c->kw;
        float *xt = nullptr, *tmp = nullptr;
        st = dalloc(s, plane * c->in_c, &xt, "conv_transpose2d staging allocation");
        if (!st) st = dalloc(s, plane * cols, &tmp, "conv_transpose2d staging allocation");
        if (!st)
            st = launch(s, "conv_transpose_to_hwc", [&] {
                return vh::launch_transpose(s.stream, input->ptr, xt, c->in_c, plane);
            });
        if (!st) st = gemm_nt(s, xt, c->w, c->bias_x, tmp, plane, cols, c->in_c, "conv_transpose_gemm");
        if (!st)
            st = launch(s, "patch_scatter", [&] {
                return vh::launch_patch_scatter(s.stream, tmp, t->ptr, c->out_c, ih, iw, c->kh, c->kw);
            });
        if (xt) hipFreeAsync(xt, s.stream);
        if (tmp) hipFreeAsync(tmp, s.stream);
    } else {
        st = launch(s, "conv_transpose_gather", [&] {
            return vh::launch_conv_transpose_gather(s.stream, input->ptr, c->w, c->bias, t->ptr,
                                                    c->in_c, ih, iw, c->out_c, c->kh, c->kw,
                                                    c->stride);
        });
    }
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

vh_status resize_new(const vh_runtime *rt, const vh_tensor *input, size_t c, size_t ih,
                     size_t iw, size_t oh, size_t ow, const vh_tensor *add, bool align,
                     vh_tensor **out, const char *name) {
    NEED(rt, name);
    NEED(input, name);
    NEED(out, name);
    size_t ilen = 0, olen = 0;
    if (mul_overflows(c, ih, &ilen) || mul_overflows(ilen, iw, &ilen) ||
        mul_overflows(c, oh, &olen) || mul_overflows(olen, ow, &olen))
        return fail(VH_ERR_KERNEL, std::string(name) + ": size overflows");
    TRY(check_tensor_len(input, ilen, name));
    if (add) TRY(check_tensor_len(add, olen, name));
    if (c > INT32_MAX || ih > INT32_MAX || iw > INT32_MAX || oh > INT32_MAX || ow > INT32_MAX ||
        (oh + 3) / 4 > 65535 || (c + 7) / 8 > 65535)
        return fail(VH_ERR_KERNEL, std::string(name) + ": shape exceeds the launch grid");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    vh_tensor *t = nullptr;
    TRY(new_tensor(rt->s, olen, &t, "resize output allocation"));
    // src/resample.rs returns without writing for an empty input or output.
    vh_status st = VH_OK;
    if (olen && ilen) {
        st = launch(s, align ? "bilinear_align_corners" : "bilinear", [&] {
            return vh::launch_bilinear(s.stream, input->ptr, add ? add->ptr : nullptr, t->ptr, c,
                                       ih, iw, oh, ow, align);
        });
    } else if (olen) {
        st = launch(s, "fill", [&] { return vh::launch_fill(s.stream, t->ptr, olen, 0.0f); });
    }
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return VH_OK;
    GUARD_END
}

}  // namespace

extern "C" vh_status vh_prepare_conv2d_f32(const vh_runtime *rt, size_t in_c, size_t out_c,
                                           size_t kh, size_t kw, size_t stride, size_t pad,
                                           const float *weight, const float *bias,
                                           vh_conv2d **out) {
    GUARD_BEGIN
    return prepare_conv(rt, in_c, out_c, kh, kw, stride, pad, weight, bias, out);
    GUARD_END
}

extern "C" void vh_conv2d_free(vh_conv2d *conv) { delete conv; }

extern "C" vh_status vh_conv2d_run(const vh_conv2d *conv, const vh_tensor *input, size_t ih,
                                   size_t iw, vh_tensor **out) {
    GUARD_BEGIN
    return conv_new(conv, input, ih, iw, false, out, "vh_conv2d_run");
    GUARD_END
}

extern "C" vh_status vh_conv2d_run_relu_input(const vh_conv2d *conv, const vh_tensor *input,
                                              size_t ih, size_t iw, vh_tensor **out) {
    GUARD_BEGIN
    return conv_new(conv, input, ih, iw, true, out, "vh_conv2d_run_relu_input");
    GUARD_END
}

extern "C" vh_status vh_conv2d_run_resize_align_corners(const vh_conv2d *conv,
                                                        const vh_tensor *input, size_t ih,
                                                        size_t iw, size_t oh, size_t ow,
                                                        const vh_tensor *add, vh_tensor **out) {
    NEED(conv, "vh_conv2d_run_resize_align_corners");
    GUARD_BEGIN
    vh_runtime rt{conv->rt};
    vh_tensor *resized = nullptr;
    TRY(resize_new(&rt, input, conv->in_c, ih, iw, oh, ow, add, true, &resized,
                   "vh_conv2d_run_resize_align_corners"));
    vh_status st = conv_new(conv, resized, oh, ow, false, out, "vh_conv2d_run_resize_align_corners");
    delete resized;
    return st;
    GUARD_END
}

extern "C" vh_status vh_conv2d_f32(const vh_runtime *rt, const vh_tensor *input, size_t in_c,
                                   size_t ih, size_t iw, const float *weight, size_t out_c,
                                   size_t kh, size_t kw, size_t stride, size_t pad,
                                   const float *bias, vh_tensor **out) {
    GUARD_BEGIN
    vh_conv2d *c = nullptr;
    TRY(prepare_conv(rt, in_c, out_c, kh, kw, stride, pad, weight, bias, &c));
    vh_status st = conv_new(c, input, ih, iw, false, out, "vh_conv2d_f32");
    delete c;
    return st;
    GUARD_END
}

extern "C" size_t vh_conv2d_output_height(const vh_conv2d *c, size_t ih) {
    return c && ih + 2 * c->pad >= c->kh ? (ih + 2 * c->pad - c->kh) / c->stride + 1 : 0;
}
extern "C" size_t vh_conv2d_output_width(const vh_conv2d *c, size_t iw) {
    return c && iw + 2 * c->pad >= c->kw ? (iw + 2 * c->pad - c->kw) / c->stride + 1 : 0;
}

extern "C" vh_status vh_prepare_conv_transpose2d_f32(const vh_runtime *rt, size_t in_c,
                                                     size_t out_c, size_t kh, size_t kw,
                                                     size_t stride, const float *weight,
                                                     const float *bias,
                                                     vh_conv_transpose2d **out) {
    GUARD_BEGIN
    return prepare_conv_t(rt, in_c, out_c, kh, kw, stride, weight, bias, out);
    GUARD_END
}

extern "C" void vh_conv_transpose2d_free(vh_conv_transpose2d *conv) { delete conv; }

extern "C" vh_status vh_conv_transpose2d_run(const vh_conv_transpose2d *conv,
                                             const vh_tensor *input, size_t ih, size_t iw,
                                             vh_tensor **out) {
    return conv_t_new(conv, input, ih, iw, out);
}

extern "C" vh_status vh_conv_transpose2d_f32(const vh_runtime *rt, const vh_tensor *input,
                                             size_t in_c, size_t ih, size_t iw,
                                             const float *weight, size_t out_c, size_t kh,
                                             size_t kw, size_t stride, const float *bias,
                                             vh_tensor **out) {
    GUARD_BEGIN
    vh_conv_transpose2d *c = nullptr;
    TRY(prepare_conv_t(rt, in_c, out_c, kh, kw, stride, weight, bias, &c));
    vh_status st = conv_t_new(c, input, ih, iw, out);
    delete c;
    return st;
    GUARD_END
}

extern "C" vh_status vh_bilinear_resize_f32(const vh_runtime *rt, const vh_tensor *input,
                                            size_t c, size_t ih, size_t iw, size_t oh, size_t ow,
                                            vh_tensor **out) {
    return resize_new(rt, input, c, ih, iw, oh, ow, nullptr, false, out, "vh_bilinear_resize_f32");
}

extern "C" vh_status vh_bilinear_resize_align_corners_f32(const vh_runtime *rt,
                                                          const vh_tensor *input, size_t c,
                                                          size_t ih, size_t iw, size_t oh,
                                                          size_t ow, const vh_tensor *add,
                                                          vh_tensor **out) {
    return resize_new(rt, input, c, ih, iw, oh, ow, add, true, out,
                      "vh_bilinear_resize_align_corners_f32");
}

// =============================================================================
// profiling
// =============================================================================

extern "C" vh_status vh_profile_enable(vh_runtime *rt, int enabled) {
    NEED(rt, "vh_profile_enable");
    rt->s->profile = enabled != 0;
    return VH_OK;
}

extern "C" vh_status vh_profile_reset(vh_runtime *rt) {
    NEED(rt, "vh_profile_reset");
    RtState &s = *rt->s;
    TRY(set_device(s));
    hipStreamSynchronize(s.stream);
    for (auto &p : s.pending) {
        hipEventDestroy(p.a);
        hipEventDestroy(p.b);
    }
    s.pending.clear();
    s.totals.clear();
    return VH_OK;
}

extern "C" vh_status vh_profile_report(vh_runtime *rt, char *buf, size_t buflen) {
    NEED(rt, "vh_profile_report");
    if (buflen && !buf) return null_arg("vh_profile_report buf");
    GUARD_BEGIN
    RtState &s = *rt->s;
    TRY(set_device(s));
    hipError_t e = hipStreamSynchronize(s.stream);
    if (e != hipSuccess) return fail(VH_ERR_KERNEL, hip_msg("profile synchronize", e));
    for (auto &p : s.pending) {
        float ms = 0.0f;
        hipEventElapsedTime(&ms, p.a, p.b);
        auto &t = s.totals[p.name];
        t.first += 1;
        t.second += ms;
        hipEventDestroy(p.a);
        hipEventDestroy(p.b);
    }
    s.pending.clear();
    std::string out;
    char line[256];
    for (auto &kv : s.totals) {
        std::snprintf(line, sizeof(line), "%s %llu %.6f\n", kv.first.c_str(), kv.second.first,
                      kv.second.second);
        out += line;
    }
    if (buflen) {
        size_t n = out.size() < buflen - 1 ? out.size() : buflen - 1;
        std::memcpy(buf, out.data(), n);
        buf[n] = '\0';
    }
    return VH_OK;
    GUARD_END
}

extern "C" vh_status vh_timer_start(vh_runtime *rt) {
    NEED(rt, "vh_timer_start");
    RtState &s = *rt->s;
    TRY(set_device(s));
    if (!s.t0 && hipEventCreate(&s.t0) != hipSuccess) return fail(VH_ERR_KERNEL, "event create");
    if (!s.t1 && hipEventCreate(&s.t1) != hipSuccess) return fail(VH_ERR_KERNEL, "event create");
    hipError_t e = hipEventRecord(s.t0, s.stream);
    if (e != hipSuccess) return fail(VH_ERR_KERNEL, hip_msg("event record", e));
    return VH_OK;
}

extern "C" vh_status vh_timer_stop(vh_runtime *rt, float *elapsed_ms) {
    NEED(rt, "vh_timer_stop");
    NEED(elapsed_ms, "vh_timer_stop");
    RtState &s = *rt->s;
    if (!s.t0) return fail(VH_ERR_KERNEL, "vh_timer_stop without vh_timer_start");
    TRY(set_device(s));
    hipError_t e = hipEventRecord(s.t1, s.stream);
    if (e == hipSuccess) e = hipEventSynchronize(s.t1);
    if (e == hipSuccess) e = hipEventElapsedTime(elapsed_ms, s.t0, s.t1);
    if (e != hipSuccess) return fail(VH_ERR_KERNEL, hip_msg("timer", e));
    return VH_OK;
}
