// gsd_capi.hip -- C ABI of libgsdhip.so (declared in include/gsdhip.h):
// operator twins of the reference CPU engine and the model runtime that runs
// a whole token as one HIP graph.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "gsd_internal.h"
#include "../../include/gsdhip.h"

using namespace gsd;

namespace {
thread_local std::string g_err;
}

namespace gsd {
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code ? code : -1;
}
void attention_test_knobs(AttnArgs& a) {
    const char* s = std::getenv("GSD_ATTN_TEST_SKEW");
    a.wait_skew = s ? std::atoi(s) : 0;
    s = std::getenv("GSD_ATTN_SPIN_LIMIT");
    a.spin_limit = s ? std::atoi(s) : 0;
}
}  // namespace gsd

namespace {


#define HIPCHK(expr)                                                                        \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess) return fail((int)e_, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Codebook of radius R as float2 (gsd_lq_cpu_runtime.py:111-118).
std::vector<float> host_table(int R) {
    std::vector<float> t;
    const double s32 = std::sqrt(3.0) / 2.0;
    for (int a = -R; a <= R; a++)
        for (int b = -R; b <= R; b++) {
            if (std::abs(a + b) > R) continue;
            t.push_back((float)((double)a + 0.5 * (double)b));
            t.push_back((float)((double)b * s32));
        }
    return t;
}

// Integer fields (r0, r1) of the radius-R codewords in enumeration order, as
// fp16 pairs (low half r0): the lattice form of the same table.
uint16_t half_of_small_int(int n) {
    if (n == 0) return 0;
    const uint16_t sign = n < 0 ? 0x8000u : 0u;
    unsigned a = (unsigned)(n < 0 ? -n : n), e = 0;
    while ((a >> (e + 1)) != 0) e++;
    const unsigned mant = (a << (10 - e)) & 0x3FFu;
    return (uint16_t)(sign | ((e + 15u) << 10) | mant);
}

std::vector<uint32_t> host_fields(int R) {
    std::vector<uint32_t> t;
    for (int a = -R; a <= R; a++)
        for (int b = -R; b <= R; b++) {
            if (std::abs(a + b) > R) continue;
            t.push_back((uint32_t)half_of_small_int(a) | ((uint32_t)half_of_small_int(b) << 16));
        }
    return t;
}

// RoPE angles exactly as gsd_lq_cpu_engine.c:213-218 evaluates them (C library
// powf/cosf/sinf in float), so the device rotation sees identical cos/sin.
__attribute__((noinline)) void rope_cs(float theta, int hd, int pos, float* out /* 2*hd/2 */) {
    const int half = hd / 2;
    for (int i = 0; i < half; i++) {
        const float freq = 1.0f / powf(theta, (float)(2 * i) / (float)hd);
        const float ang = (float)pos * freq;
        out[2 * i] = cosf(ang);
        out[2 * i + 1] = sinf(ang);
    }
}

// Workspaces of the attention twins that a caller created for a stream
// (gsdh_attention_workspace_create): calls on such a stream use it, calls on
// other streams the library's per-device static scratch.  Each holds the
// 256-byte header (device epoch word, error word) and the split words; the
// epoch lives on the device, so the host keeps no per-launch state.
struct AttnWs {
    unsigned long long* ws = nullptr;   // header + words
    size_t bytes = 0;                   // words only
    int dev = 0;
};
std::mutex g_attn_mu;
std::map<hipStream_t, AttnWs> g_attn_ws;


}  // namespace

extern "C" {

const char* gsdh_last_error(void) { return g_err.c_str(); }

int gsdh_device_info(char* name, int name_len, uint64_t* total_bytes, int* n_cu) {
    int dev = 0;
    HIPCHK(hipGetDevice(&dev));
    hipDeviceProp_t p;
    HIPCHK(hipGetDeviceProperties(&p, dev));
    if (name && name_len > 0) {
        snprintf(name, name_len, "%s (%s)", p.name[0] ? p.name : "AMD Instinct", p.gcnArchName);
    }
    if (total_bytes) *total_bytes = p.totalGlobalMem;
    if (n_cu) *n_cu = p.multiProcessorCount;
    return 0;
}

int gsdh_malloc(void** ptr, uint64_t nbytes) {
    HIPCHK(hipMalloc(ptr, nbytes ? nbytes : 4));
    return 0;
}
int gsdh_free(void* ptr) {
    HIPCHK(hipFree(ptr));
    return 0;
}
int gsdh_memcpy_h2d(void* dst, const void* src, uint64_t n, void* stream) {
    HIPCHK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, S(stream)));
    return 0;
}
int gsdh_memcpy_d2h(void* dst, const void* src, uint64_t n, void* stream) {
    HIPCHK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, S(stream)));
    return 0;
}
int gsdh_stream_copy(void* stream, void* dst, const void* src, uint64_t nbytes) {
    HIPCHK(launch_copy(src, dst, nbytes, S(stream)));
    return 0;
}
int gsdh_stream_sync(void* stream) {
    HIPCHK(hipStreamSynchronize(S(stream)));
    // a stand-alone attention launch whose merge gave up waiting for a
    // split's partials (bounded wait) left its error word set: report it
    // here, as an asynchronous failure surfaces at the next synchronisation
    int bad = 0;
    int rc = attention_static_error(&bad);
    if (rc) return rc;
    unsigned* ew = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_attn_mu);
        auto it = g_attn_ws.find(S(stream));
        if (it != g_attn_ws.end()) ew = reinterpret_cast<unsigned*>(it->second.ws + 1);
    }
    if (ew) {
        unsigned v = 0;
        HIPCHK(hipMemcpy(&v, ew, 4, hipMemcpyDeviceToHost));
        if (v) {
            const unsigned zero = 0;
            HIPCHK(hipMemcpy(ew, &zero, 4, hipMemcpyHostToDevice));
            bad = 1;
        }
    }
    if (bad)
        return fail(-2, "stream_sync: an attention launch's merge timed out waiting for split partials "
                        "(its output is undefined)");
    return 0;
}

int gsdh_stream_create(void** stream_out) {
    if (!stream_out) return fail(-1, "stream_create: null argument");
    hipStream_t s = nullptr;
    HIPCHK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream_out = s;
    return 0;
}

int gsdh_stream_destroy(void* stream) {
    if (!stream) return 0;
    HIPCHK(hipStreamSynchronize(S(stream)));
    int rc = gsdh_attention_workspace_destroy(stream);
    if (rc) return rc;
    HIPCHK(hipStreamDestroy(S(stream)));
    return 0;
}

int gsdh_stream_begin_capture(void* stream) {
    HIPCHK(hipStreamBeginCapture(S(stream), hipStreamCaptureModeThreadLocal));
    return 0;
}

int gsdh_stream_end_capture(void* stream, void** graph_exec_out) {
    if (!graph_exec_out) return fail(-1, "stream_end_capture: null argument");
    hipGraph_t g = nullptr;
    HIPCHK(hipStreamEndCapture(S(stream), &g));
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return fail((int)e, "hipGraphInstantiate: %s", hipGetErrorString(e));
    *graph_exec_out = ge;
    return 0;
}

int gsdh_graph_replay(void* graph_exec, void* stream) {
    HIPCHK(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph_exec), S(stream)));
    return 0;
}

uint64_t gsdh_attention_workspace_bytes(int n_kv_heads, int n_heads, int head_dim, int max_seq_len) {
    if (n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads || head_dim <= 0 || max_seq_len <= 0) return 0;
    return kAttnWsHeader + attention_ws_bytes_upto(n_kv_heads, n_heads / n_kv_heads, head_dim, max_seq_len);
}

int gsdh_attention_workspace_create(void* stream, int n_kv_heads, int n_heads, int head_dim, int max_seq_len) {
    const uint64_t total = gsdh_attention_workspace_bytes(n_kv_heads, n_heads, head_dim, max_seq_len);
    if (!total) return fail(-1, "attention_workspace_create: n_kv_heads %d n_heads %d head_dim %d max_seq_len %d",
                            n_kv_heads, n_heads, head_dim, max_seq_len);
    int rc = gsdh_attention_workspace_destroy(stream);
    if (rc) return rc;
    AttnWs w;
    HIPCHK(hipGetDevice(&w.dev));
    HIPCHK(hipMalloc(&w.ws, total));
    w.bytes = total - kAttnWsHeader;
    hipError_t e = launch_fill_u32(reinterpret_cast<unsigned*>(w.ws), 0u, total / 4, S(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(S(stream));
    if (e != hipSuccess) {
        (void)hipFree(w.ws);
        return fail((int)e, "attention_workspace_create: %s", hipGetErrorString(e));
    }
    std::lock_guard<std::mutex> lk(g_attn_mu);
    g_attn_ws[S(stream)] = w;
    return 0;
}

int gsdh_attention_workspace_destroy(void* stream) {
    AttnWs w;
    {
        std::lock_guard<std::mutex> lk(g_attn_mu);
        auto it = g_attn_ws.find(S(stream));
        if (it == g_attn_ws.end()) return 0;
        w = it->second;
        g_attn_ws.erase(it);
    }
    HIPCHK(hipStreamSynchronize(S(stream)));
    HIPCHK(hipFree(w.ws));
    return 0;
}

// ---------------------------------------------------------------------------
// operator twins
// ---------------------------------------------------------------------------
int gsdh_rmsnorm(void* stream, const float* x, const float* w, float* out, int dim, float eps) {
    if (dim <= 0) return fail(-1, "rmsnorm: dim %d", dim);
    HIPCHK(launch_rmsnorm(x, w, out, dim, eps, S(stream)));
    return 0;
}

int gsdh_vec_add(void* stream, float* y, const float* a, const float* b, int dim) {
    HIPCHK(launch_vec_add(y, a, b, dim, S(stream)));
    return 0;
}

int gsdh_swiglu(void* stream, const float* g, const float* u, float* out, int dim) {
    HIPCHK(launch_swiglu(g, u, out, dim, S(stream)));
    return 0;
}

int gsdh_lowrank_proj(void* stream, const float* x, const uint16_t* Vt, const float* Sv, float* tmp_k,
                      int k_dim, int cols) {
    if (k_dim < 0 || k_dim > kMaxRank) return fail(-1, "lowrank_proj: k_dim %d outside 0..%d", k_dim, kMaxRank);
    HIPCHK(launch_lowrank(x, Vt, Sv, tmp_k, k_dim, cols, S(stream)));
    return 0;
}

int gsdh_hex2d_matvec(void* stream, const float* x, const uint8_t* codes, const uint16_t* scales,
                      const float* xy_table, const uint16_t* U, const float* tmp_k, const uint32_t* kink_row_ptr,
                      const uint16_t* kink_cols, const float* kink_deltas, float* y, int rows, int cols, int k_dim,
                      int n_pts) {
    if (rows < 0) return fail(-1, "hex2d_matvec: rows %d", rows);
    if (cols <= 0 || cols % 64) return fail(-1, "hex2d_matvec: cols %d is not a positive multiple of 64", cols);
    if (cols > 65536) return fail(-1, "hex2d_matvec: cols %d > 65536", cols);
    if (k_dim < 0 || k_dim > kMaxRank) return fail(-1, "hex2d_matvec: k_dim %d outside 0..%d", k_dim, kMaxRank);
    if (n_pts <= 0 || n_pts > kTableSlots) return fail(-1, "hex2d_matvec: n_pts %d outside 1..256", n_pts);
    if (k_dim > 0 && (!U || !tmp_k)) return fail(-1, "hex2d_matvec: k_dim > 0 needs U and tmp_k");
    HexArgs a{};
    a.nseg = 1;
    HexSeg& s = a.seg[0];
    s.codes = codes; s.scales = scales; s.row_ptr = kink_row_ptr; s.kcols = kink_cols; s.kdel = kink_deltas;
    s.U = U; s.Vt = nullptr; s.S = nullptr; s.tmp_k = tmp_k; s.table = xy_table; s.out = y;
    s.rows = rows; s.k = k_dim; s.n_pts = n_pts;
    a.x = x; a.norm_w = nullptr; a.eps = 0.f; a.resid = nullptr; a.cols = cols; a.epilogue = kEpiStore;
    HIPCHK(launch_hexmv(a, S(stream)));
    return 0;
}

int gsdh_rope_and_store_kv(void* stream, float* q, const float* k, const float* v, uint16_t* k_cache,
                           uint16_t* v_cache, int layer_idx, int pos, int n_heads, int n_kv_heads, int head_dim,
                           int max_seq_len, float rope_theta, int interleaved) {
    if (head_dim <= 0 || head_dim % 2 || head_dim > 256) return fail(-1, "rope: head_dim %d", head_dim);
    if (pos < 0 || pos >= max_seq_len) return fail(-1, "rope: pos %d outside 0..%d", pos, max_seq_len - 1);
    std::vector<float> cs(head_dim);
    rope_cs(rope_theta, head_dim, pos, cs.data());
    RopeKV r{};
    r.cs = nullptr; r.pos_dev = nullptr; r.pos = pos; r.k_cache = k_cache; r.v_cache = v_cache;
    r.layer = layer_idx; r.n_heads = n_heads; r.n_kv = n_kv_heads; r.hd = head_dim; r.max_seq = max_seq_len;
    r.interleaved = interleaved;
    HIPCHK(launch_rope_kv(q, k, v, r, reinterpret_cast<const float2*>(cs.data()), S(stream)));
    return 0;
}

namespace {
// Checks a one-token attention call and fills a (positions, chunking, and the
// workspace: the stream's own, else the library's static scratch); nothing
// is allocated.
int attention_setup(void* stream, AttnArgs& a, const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                    float* attn_out, int layer_idx, int pos, int n_heads, int n_kv_heads, int head_dim,
                    int max_seq_len, float sm_scale) {
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return fail(-1, "attention: head_dim %d not in {64,128,256}", head_dim);
    if (n_kv_heads <= 0 || n_heads % n_kv_heads || (8 % (n_heads / n_kv_heads)) != 0)
        return fail(-1, "attention: n_heads %d / n_kv_heads %d is not a group size in {1,2,4,8}", n_heads, n_kv_heads);
    if (pos < 0 || pos >= max_seq_len) return fail(-1, "attention: pos %d outside 0..%d", pos, max_seq_len - 1);
    const int n = pos + 1, G = n_heads / n_kv_heads;
    a = AttnArgs{};
    a.q = q; a.k_cache = k_cache; a.v_cache = v_cache; a.out = attn_out; a.pos_dev = nullptr; a.pos = pos;
    a.layer = layer_idx; a.n_heads = n_heads; a.n_kv = n_kv_heads; a.hd = head_dim; a.max_seq = max_seq_len;
    a.sm_scale = sm_scale;
    a.chunk = attention_chunk(n, n_kv_heads);
    a.max_splits = (n + a.chunk - 1) / a.chunk;
    attention_test_knobs(a);
    const size_t need = attention_ws_bytes(n_kv_heads, a.max_splits, G, head_dim);
    {
        std::lock_guard<std::mutex> lk(g_attn_mu);
        auto it = g_attn_ws.find(S(stream));
        if (it != g_attn_ws.end()) {
            if (need > it->second.bytes)
                return fail(-1, "attention: %zu bytes of split partials exceed the stream's workspace (%zu bytes); "
                                "create it for a longer context", need, it->second.bytes);
            attention_use_ws(a, it->second.ws);
            return 0;
        }
    }
    return attention_static_ws(S(stream), a, G, "attention");
}
}  // namespace

int gsdh_gqa_attention(void* stream, const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                       float* attn_out, int layer_idx, int pos, int n_heads, int n_kv_heads, int head_dim,
                       int max_seq_len, float sm_scale) {
    AttnArgs a;
    const int rc = attention_setup(stream, a, q, k_cache, v_cache, attn_out, layer_idx, pos, n_heads, n_kv_heads,
                                   head_dim, max_seq_len, sm_scale);
    if (rc) return rc;
    HIPCHK(launch_attention(a, S(stream)));
    return 0;
}

int gsdh_prefill_attention(void* stream, const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                           float* attn_out, int layer_idx, int pos0, int n_tokens, int n_heads, int n_kv_heads,
                           int head_dim, int max_seq_len, float sm_scale) {
    if (n_tokens < 0 || pos0 < 0 || layer_idx < 0 || max_seq_len <= 0 || pos0 + n_tokens > max_seq_len)
        return fail(-1, "prefill_attention: %d tokens at %d, max_seq_len %d", n_tokens, pos0, max_seq_len);
    if (n_kv_heads <= 0 || n_heads % n_kv_heads || 8 % (n_heads / n_kv_heads))
        return fail(-1, "prefill_attention: %d query heads over %d KV heads", n_heads, n_kv_heads);
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return fail(-1, "prefill_attention: head_dim %d not in {64,128,256}", head_dim);
    if (n_tokens && (!q || !k_cache || !v_cache || !attn_out)) return fail(-1, "prefill_attention: null buffer");
    PrefillAttn a{};
    a.q = q; a.k_cache = k_cache; a.v_cache = v_cache; a.out = attn_out; a.layer = layer_idx; a.p0 = pos0;
    a.M = n_tokens; a.n_heads = n_heads; a.n_kv = n_kv_heads; a.hd = head_dim; a.max_seq = max_seq_len;
    a.sm_scale = sm_scale;
    HIPCHK(launch_prefill_attention(a, S(stream)));
    return 0;
}

int gsdh_rope_store_gqa_attention(void* stream, float* q, const float* k, const float* v, uint16_t* k_cache,
                                  uint16_t* v_cache, float* attn_out, int layer_idx, int pos, int n_heads,
                                  int n_kv_heads, int head_dim, int max_seq_len, float rope_theta, int interleaved,
                                  float sm_scale) {
    if (head_dim <= 0 || head_dim % 2 || head_dim > 256) return fail(-1, "rope: head_dim %d", head_dim);
    AttnArgs a;
    const int rc = attention_setup(stream, a, q, k_cache, v_cache, attn_out, layer_idx, pos, n_heads, n_kv_heads,
                                   head_dim, max_seq_len, sm_scale);
    if (rc) return rc;
    std::vector<float> cs(head_dim);
    rope_cs(rope_theta, head_dim, pos, cs.data());
    const float2* cs2 = reinterpret_cast<const float2*>(cs.data());
    const hipError_t e = launch_rope_attention(a, k, v, interleaved, cs2, S(stream));
    if (e == hipSuccess) return 0;
    if (e != hipErrorNotSupported) return fail((int)e, "rope + attention: %s", hipGetErrorString(e));
    // shapes outside the fused kernel: the two launches
    RopeKV r{};
    r.cs = nullptr; r.pos_dev = nullptr; r.pos = pos; r.k_cache = k_cache; r.v_cache = v_cache;
    r.layer = layer_idx; r.n_heads = n_heads; r.n_kv = n_kv_heads; r.hd = head_dim; r.max_seq = max_seq_len;
    r.interleaved = interleaved;
    HIPCHK(launch_rope_kv(q, k, v, r, cs2, S(stream)));
    HIPCHK(launch_attention(a, S(stream)));
    return 0;
}

int gsdh_unpack_codes(void* stream, const uint8_t* codes, int64_t n, int radius, int32_t* idx_out, int8_t* r01_out) {
    if (radius < 1 || radius > 8) return fail(-1, "unpack: radius %d outside 1..8", radius);
    HIPCHK(launch_unpack(codes, n, radius, idx_out, r01_out, S(stream)));
    return 0;
}

int gsdh_greedy_argmax(void* stream, const float* logits, int n, int* token_out, float* margin_out) {
    if (n <= 0) return fail(-1, "argmax: n %d", n);
    if (!logits || !token_out || !margin_out) return fail(-1, "argmax: null argument");
    HIPCHK(launch_argmax(logits, n, nullptr, token_out, margin_out, 0, S(stream)));
    return 0;
}

int gsdh_greedy_argmax_split(void* stream, const float* logits, int n, int* token_out, float* margin_out,
                             uint64_t* words, uint32_t* counters) {
    if (n <= 0) return fail(-1, "argmax_split: n %d", n);
    if (!logits || !token_out || !margin_out || !words || !counters) return fail(-1, "argmax_split: null argument");
    HIPCHK(launch_argmax(logits, n, nullptr, token_out, margin_out, 0, S(stream),
                         reinterpret_cast<unsigned long long*>(words), counters));
    return 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// model runtime
// ---------------------------------------------------------------------------
namespace {
constexpr int kMatmulMaxM = 512;    // tokens per gsdh_model_matmul call
// prompt tokens per batched prefill pass: the projections' matrix-core tiles
// need a few hundred tokens to pass the latency bound (7B Turbo layer set:
// 1.6 us per token at 128 tokens, 0.78 at 512)
constexpr int kPrefillChunk = 512;
}  // namespace

struct HexDev {
    int set = 0, radius = 0, rows = 0, cols = 0, k = 0;
    int64_t nk = 0;
    uint4* codes_t = nullptr;      // tiled layout (HexSeg::codes_t)
    uint32_t* scales_t = nullptr;  // tiled layout (HexSeg::scales_t)
    uint32_t* row_ptr = nullptr;
    uint16_t* kcols = nullptr;
    float* kdel = nullptr;
    uint16_t* U = nullptr;
    float* Sv = nullptr;
    uint16_t* Vt = nullptr;
    // down only: the column slabs of the fused FFN launch (FfnArgs::dcodes)
    unsigned char* dslab = nullptr;
    uint32_t* dslab_sc = nullptr;
    void* block = nullptr;
    size_t bytes = 0;
};

struct gsdh_model {
    gsdh_model_config c{};
    hipStream_t stream = nullptr;
    float* tables[9] = {};          // by radius: codeword points
    uint32_t* fields[9] = {};       // by radius: (r0, r1) fp16 pairs
    uint16_t* embed = nullptr;
    float* norms = nullptr;         // [n_layers][2][hidden] + output [hidden]
    std::vector<HexDev> hex;        // n_layers * 7 + 1
    float *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *h = nullptr, *logits = nullptr;
    uint16_t *kc = nullptr, *vc = nullptr;
    float2* cs = nullptr;
    unsigned long long* ws = nullptr;   // attention partial words
    unsigned* counters = nullptr;
    // batched work, allocated at finalize (the calls allocate nothing):
    // gsdh_model_matmul staging (A fragments | descales | rank-k values |
    // split partials) for up to kMatmulMaxM tokens, and the prefill buffers
    // for chunks of up to kPrefillChunk prompt tokens
    void* mm_ws = nullptr;
    size_t mm_ws_bytes = 0;
    struct Prefill {
        int* tok = nullptr;                       // [chunk] token ids
        float *X = nullptr, *Q = nullptr, *K = nullptr, *V = nullptr, *A = nullptr, *G = nullptr, *U = nullptr;
        float* xn = nullptr;                      // prepared input [chunk][max cols]
        uint4* xa = nullptr;                      // hi/lo MFMA fragments
        float* xs = nullptr;                      // per-token descales
        float* tmp = nullptr;                     // rank-k values [kMaxSeg][chunk][kMaxRank]
        float* part = nullptr;                    // split partials
        size_t part_bytes = 0;
        int chunk = 0;
        bool batched = true;                      // generate_greedy prefills in batches
    } pf;
    unsigned long long* pub = nullptr;   // rank-k publication words, one range per matvec launch
    int pub_words = 0, pub_next = 0;
    // decode attention inside the q/k/v launch (short-context graphs): the
    // q/k/v hand-off words [qd + kvd] and the token counter that tags them
    unsigned long long* fa_words = nullptr;
    unsigned* fa_epoch = nullptr;
    bool fa_on = true;                   // GSD_FUSED_ATTN=0 turns it off (A/B)
    // the greedy step's hand-off words and per-block launch counters
    unsigned long long* am_words = nullptr;
    unsigned* am_ctr = nullptr;
    // the fused FFN launch (gate/up + SwiGLU + down + residual): its partial
    // words and per-block launch counters
    unsigned long long* ffn_words = nullptr;
    unsigned* ffn_ctr = nullptr;
    bool ffn_on = true;                  // GSD_FUSED_FFN=0 turns it off (A/B)
    bool offn_on = true;                 // the o projection in the same launch (GSD_FUSED_OFFN=0: off)
    int chunk = 64, max_splits = 1;
    StepState* st = nullptr;        // device
    StepState* st_host = nullptr;   // pinned
    int* gen_tok = nullptr;
    float* gen_margin = nullptr;
    // per-token graphs: with and without the lm_head / argmax, for any
    // position (split attention + merge) and, for positions below 64, 128
    // and 256, one attention block per KV head whose chunk is that size (it
    // loads the chunk's rows before it reads the position)
    hipGraphExec_t g_full = nullptr, g_prefill = nullptr;
    hipGraphExec_t g_full_s[kShortTiers] = {}, g_prefill_s[kShortTiers] = {};
    hipGraph_t capture_graph = nullptr;
    size_t dev_bytes = 0;
    bool finalized = false;
    std::vector<void*> allocs;

    HexDev& slot(int layer, int s) { return s == GSDH_LM_HEAD ? hex.back() : hex[(size_t)layer * 7 + s]; }
    float* norm(int layer, int which) {
        return layer < 0 ? norms + (size_t)c.n_layers * 2 * c.hidden : norms + ((size_t)layer * 2 + which) * c.hidden;
    }
};

namespace {

int dalloc(gsdh_model* m, void** p, size_t n) {
    hipError_t e = hipMalloc(p, n ? n : 4);
    if (e != hipSuccess) return fail((int)e, "hipMalloc(%zu): %s", n, hipGetErrorString(e));
    m->allocs.push_back(*p);
    m->dev_bytes += n;
    return 0;
}

void fill_seg(HexSeg& s, const HexDev& t, const gsdh_model* m, float* out) {
    s.codes_t = t.codes_t; s.scales_t = t.scales_t; s.row_ptr = t.nk ? t.row_ptr : nullptr;
    s.kcols = t.kcols; s.kdel = t.kdel; s.U = t.U; s.Vt = t.Vt; s.S = t.Sv; s.tmp_k = nullptr;
    s.table = m->tables[t.radius]; s.fields = m->fields[t.radius]; s.out = out; s.rows = t.rows; s.k = t.k;
    s.n_pts = 3 * t.radius * t.radius + 3 * t.radius + 1;
}

// Rank-k segments publish their projections inside the matvec launch (blocks
// 0..sum(k)-1): give the launch the next sum(k) publication words of the
// sequence (zeroed at its start) and the error word.
int prep_lowrank(gsdh_model* m, HexArgs& a) {
    int nlead = 0;
    for (int g = 0; g < a.nseg; g++) nlead += a.seg[g].k;
    if (nlead == 0) return 0;
    if (m->pub_next + nlead > m->pub_words)
        return fail(-1, "rank-k publication words exhausted (%d + %d > %d)", m->pub_next, nlead, m->pub_words);
    a.pub = m->pub + m->pub_next;
    a.err = &m->st->err;
    m->pub_next += nlead;
    return 0;
}

// q, k, v of layer l: fused attention RMSNorm; interleaved RoPE + KV append in the epilogue
HexArgs qkv_args(gsdh_model* m, int l) {
    const auto& c = m->c;
    HexArgs a{};
    a.nseg = 3;
    fill_seg(a.seg[0], m->slot(l, GSDH_Q), m, m->q);
    fill_seg(a.seg[1], m->slot(l, GSDH_K), m, m->k);
    fill_seg(a.seg[2], m->slot(l, GSDH_V), m, m->v);
    a.x = m->x; a.norm_w = m->norm(l, 0); a.eps = c.rms_eps; a.cols = c.hidden; a.epilogue = kEpiStore;
    a.scale_t = 1;
    if (c.rope_interleaved) {
        a.epilogue = kEpiRopeKV;
        RopeKV& r = a.rope;
        r.cs = m->cs; r.pos_dev = &m->st->pos; r.k_cache = m->kc; r.v_cache = m->vc; r.layer = l;
        r.n_heads = c.n_heads; r.n_kv = c.n_kv_heads; r.hd = c.head_dim; r.max_seq = c.max_seq_len;
        r.interleaved = 1;
    }
    return a;
}

// q, k, v of layer l and the decode attention of positions < 256 in one
// launch (sets *fused); *fused = false, with nothing launched, where the
// fused kernel does not cover the model (the caller then issues the two).
int issue_qkv_attention(gsdh_model* m, int l, int span, bool* fused) {
    const auto& c = m->c;
    *fused = false;
    if (!m->fa_on || !m->fa_words || !c.rope_interleaved) return 0;
    HexArgs a = qkv_args(m, l);
    const int pub0 = m->pub_next;
    int rc = prep_lowrank(m, a);
    if (rc) return rc;
    a.fa.words = m->fa_words; a.fa.out = m->attn; a.fa.epoch_dev = m->fa_epoch;
    a.fa.sm_scale = 1.0f / (float)std::sqrt((double)c.head_dim);
    a.fa.nkv = c.n_kv_heads;
    a.fa.span = span;
    a.err = &m->st->err;
    const hipError_t e = launch_hexmv4(a, m->stream);
    if (e == hipErrorNotSupported) {
        m->pub_next = pub0;   // (nothing launched: the two-launch path takes these words)
        return 0;
    }
    HIPCHK(e);
    *fused = true;
    return 0;
}

// Whether layer l's gate/up + down run as one fused FFN launch: the model
// shape within launch_ffn's grid, one codebook for the three tensors, and
// rank 2 in each (Precision) or in none (Turbo).
bool ffn_fused(gsdh_model* m, int l) {
    if (!m->ffn_on) return false;
    const HexDev& g = m->slot(l, GSDH_GATE);
    const HexDev& u = m->slot(l, GSDH_UP);
    const HexDev& d = m->slot(l, GSDH_DOWN);
    if (!d.dslab || g.radius != u.radius || g.radius != d.radius) return false;
    return (g.k == 0 && u.k == 0 && d.k == 0) || (g.k == 2 && u.k == 2 && d.k == 2);
}

// Whether layer l's o projection runs in the same launch as its FFN: the FFN
// fused, o of the FFN's radius and rank, o square (n_heads * head_dim ==
// hidden: its input chunks are the FFN's).
bool offn_fused(gsdh_model* m, int l) {
    if (!m->offn_on || !ffn_fused(m, l)) return false;
    const HexDev& o = m->slot(l, GSDH_O);
    const HexDev& g = m->slot(l, GSDH_GATE);
    return o.radius == g.radius && o.k == g.k && o.cols == o.rows;
}

int issue_ffn(gsdh_model* m, int l, bool with_o) {
    const auto& c = m->c;
    const HexDev& g = m->slot(l, GSDH_GATE);
    const HexDev& u = m->slot(l, GSDH_UP);
    const HexDev& d = m->slot(l, GSDH_DOWN);
    FfnArgs a{};
    a.gcodes = reinterpret_cast<const unsigned char*>(g.codes_t); a.gscales = g.scales_t;
    a.ucodes = reinterpret_cast<const unsigned char*>(u.codes_t); a.uscales = u.scales_t;
    a.dcodes = d.dslab; a.dscales = d.dslab_sc;
    a.fields = m->fields[g.radius];
    a.n_pts = 3 * g.radius * g.radius + 3 * g.radius + 1;
    if (g.nk) { a.g_rp = g.row_ptr; a.g_kc = g.kcols; a.g_kd = g.kdel; }
    if (u.nk) { a.u_rp = u.row_ptr; a.u_kc = u.kcols; a.u_kd = u.kdel; }
    if (d.nk) { a.d_rp = d.row_ptr; a.d_kc = d.kcols; a.d_kd = d.kdel; }
    if (g.k == 2) {
        a.gU = g.U; a.uU = u.U; a.dU = d.U;
        a.gS = g.Sv; a.uS = u.Sv; a.dS = d.Sv;
        a.gVt = g.Vt; a.uVt = u.Vt; a.dVt = d.Vt;
    }
    if (with_o) {
        const HexDev& o = m->slot(l, GSDH_O);
        a.ocodes = reinterpret_cast<const unsigned char*>(o.codes_t); a.oscales = o.scales_t;
        if (o.nk) { a.o_rp = o.row_ptr; a.o_kc = o.kcols; a.o_kd = o.kdel; }
        if (o.k == 2) { a.oU = o.U; a.oS = o.Sv; a.oVt = o.Vt; }
        a.attn = m->attn;
        a.qd = o.cols;
    }
    a.x = m->x; a.norm_w = m->norm(l, 1); a.eps = c.rms_eps; a.h = m->h;
    a.words = m->ffn_words; a.ctr = m->ffn_ctr; a.err = &m->st->err;
    a.hidden = c.hidden; a.ffn = c.ffn;
    HIPCHK(launch_ffn(a, m->stream));
    return 0;
}

int issue_linear(gsdh_model* m, int l, int mask) {
    int rc = 0;
    // gate/up and down together: one fused FFN launch where it covers the
    // layer, with o in it too where o is issued with them
    const bool fffn = (mask & 12) == 12 && ffn_fused(m, l);
    const bool fo = fffn && (mask & 2) && offn_fused(m, l);
    if (mask & 1) {
        HexArgs a = qkv_args(m, l);
        if ((rc = prep_lowrank(m, a))) return rc;
        HIPCHK(launch_hexmv4(a, m->stream));
    }
    const auto& c = m->c;
    if ((mask & 2) && !fo) {   // o projection + residual
        HexArgs a{};
        a.nseg = 1;
        fill_seg(a.seg[0], m->slot(l, GSDH_O), m, m->x);
        a.x = m->attn; a.cols = c.n_heads * c.head_dim; a.epilogue = kEpiResidual; a.resid = m->x;
        a.scale_t = 1;
        if ((rc = prep_lowrank(m, a))) return rc;
        HIPCHK(launch_hexmv4(a, m->stream));
    }
    if (fffn) return issue_ffn(m, l, fo);
    if (mask & 4) {   // gate + up with fused FFN RMSNorm and SwiGLU
        HexArgs a{};
        a.nseg = 2;
        fill_seg(a.seg[0], m->slot(l, GSDH_GATE), m, m->h);
        fill_seg(a.seg[1], m->slot(l, GSDH_UP), m, nullptr);
        a.x = m->x; a.norm_w = m->norm(l, 1); a.eps = c.rms_eps; a.cols = c.hidden; a.epilogue = kEpiSwiGLU;
        a.scale_t = 1;
        if ((rc = prep_lowrank(m, a))) return rc;
        HIPCHK(launch_hexmv4(a, m->stream));
    }
    if (mask & 8) {   // down projection + residual
        HexArgs a{};
        a.nseg = 1;
        fill_seg(a.seg[0], m->slot(l, GSDH_DOWN), m, m->x);
        a.x = m->h; a.cols = c.ffn; a.epilogue = kEpiResidual; a.resid = m->x;
        a.scale_t = 1;
        if ((rc = prep_lowrank(m, a))) return rc;
        HIPCHK(launch_hexmv4(a, m->stream));
    }
    return 0;
}

// Final RMSNorm + lm_head (run_gpu_native_chat.py:962-968) and, with
// `greedy`, the device argmax that appends the token and advances the step.
int issue_head(gsdh_model* m, bool greedy) {
    const auto& c = m->c;
    HexArgs a{};
    a.nseg = 1;
    fill_seg(a.seg[0], m->slot(0, GSDH_LM_HEAD), m, m->logits);
    a.x = m->x; a.norm_w = m->norm(-1, 0); a.eps = c.rms_eps; a.cols = c.hidden; a.epilogue = kEpiStore;
    a.scale_t = 1;
    int rc = prep_lowrank(m, a);
    if (rc) return rc;
    HIPCHK(launch_hexmv4(a, m->stream));
    if (greedy)
        HIPCHK(launch_argmax(m->logits, c.vocab, m->st, m->gen_tok, m->gen_margin, 1, m->stream, m->am_words, m->am_ctr));
    return 0;
}

// The per-token launch sequence (run_gpu_native_chat.py:892-969, fused).
// short_chunk: 0 for the graph of any position, else the single attention
// chunk (64, 128 or 256) of the graph for positions below it
int issue_token(gsdh_model* m, bool with_head, int short_chunk) {
    const auto& c = m->c;
    m->pub_next = 0;
    HIPCHK(launch_embed(m->embed, &m->st->token, m->x, c.hidden, m->pub, m->pub_words, m->fa_epoch, m->stream));
    for (int l = 0; l < c.n_layers; l++) {
        // positions < 256: the attention in the q/k/v launch where it covers the model
        bool fused = false;
        int rc = short_chunk ? issue_qkv_attention(m, l, short_chunk, &fused) : 0;
        if (rc) return rc;
        if (fused) {
            rc = issue_linear(m, l, 2 | 4 | 8);
            if (rc) return rc;
            continue;
        }
        rc = issue_linear(m, l, 1);
        if (rc) return rc;
        if (!c.rope_interleaved) {   // (i, i+hd/2) pairs are not adjacent rows: separate kernel
            RopeKV r{};
            r.cs = m->cs; r.pos_dev = &m->st->pos; r.k_cache = m->kc; r.v_cache = m->vc; r.layer = l;
            r.n_heads = c.n_heads; r.n_kv = c.n_kv_heads; r.hd = c.head_dim; r.max_seq = c.max_seq_len;
            r.interleaved = 0;
            HIPCHK(launch_rope_kv(m->q, m->k, m->v, r, nullptr, m->stream));
        }
        AttnArgs a{};
        a.q = m->q; a.k_cache = m->kc; a.v_cache = m->vc; a.out = m->attn; a.pos_dev = &m->st->pos;
        a.layer = l; a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.hd = c.head_dim; a.max_seq = c.max_seq_len;
        a.sm_scale = 1.0f / (float)std::sqrt((double)c.head_dim);
        a.chunk = m->chunk; a.max_splits = m->max_splits; a.ws = m->ws; a.counters = m->counters;
        a.err = &m->st->err;
        if (short_chunk) {   // positions < short_chunk: one block per KV head
            a.chunk = short_chunk;
            a.max_splits = 1;
        }
        HIPCHK(launch_attention(a, m->stream));
        rc = issue_linear(m, l, 2 | 4 | 8);
        if (rc) return rc;
    }
    if (with_head) return issue_head(m, true);
    return 0;
}

hipGraphExec_t token_graph(const gsdh_model* m, bool with_head, int pos) {
    for (int t = 0; t < kShortTiers; t++)
        if (pos < kShortChunk[t]) return with_head ? m->g_full_s[t] : m->g_prefill_s[t];
    return with_head ? m->g_full : m->g_prefill;
}

// Staging bytes of one gsdh_model_matmul call (bf16 X, single fp16 operand
// rounding): A fragments, descales, rank-k values (one slot per tensor of a
// shared-input call), split partials.
size_t matmul_ws_need(int M, int rows, int cols) {
    const size_t xa = (hexmm_xa_bytes(M, cols) + 255) / 256 * 256;
    const size_t xs = ((size_t)(M + 15) / 16 * 16 * 4 + 255) / 256 * 256;
    const size_t tk = ((size_t)M * kMaxRank * 4 + 255) / 256 * 256;
    const MatmulPlan plan = hexmm_plan(M, rows, cols);
    const size_t pt = plan.nsplit > 1 ? (size_t)plan.nsplit * ((M + 15) / 16 * 16) * rows * 4 : 0;
    return xa + xs + kMaxSeg * tk + pt;
}

size_t split_part_bytes(int M, int rows, int cols) {   // the prefill's (high + low operands)
    const MatmulPlan plan = hexmm_plan(M, rows, cols, true);
    return plan.nsplit > 1 ? (size_t)plan.nsplit * ((M + 15) / 16 * 16) * rows * 4 : 0;
}

// The batched workspaces, sized for every tensor shape of the model and every
// batch size up to the limits, so no later call allocates.
int setup_batched(gsdh_model* m) {
    const auto& c = m->c;
    const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    const int shapes[5][2] = {{qd, c.hidden}, {kvd, c.hidden}, {c.hidden, qd}, {c.ffn, c.hidden}, {c.hidden, c.ffn}};
    size_t mm = 0, part = 0;
    for (int M = 1; M <= kMatmulMaxM; M++) {
        for (const auto& sh : shapes) {
            mm = std::max(mm, matmul_ws_need(M, sh[0], sh[1]));
            if (M <= kPrefillChunk) part = std::max(part, split_part_bytes(M, sh[0], sh[1]));
        }
        mm = std::max(mm, matmul_ws_need(M, c.vocab, c.hidden));
    }
    auto& P = m->pf;
    const int Mc = kPrefillChunk, Mp = (Mc + 15) / 16 * 16;
    const int maxc = std::max(std::max(c.hidden, c.ffn), qd);
    P.chunk = Mc;
    P.part_bytes = part;
    int rc = 0;
    auto A = [&](void** p, size_t n) { if (!rc) rc = dalloc(m, p, n); };
    A(&m->mm_ws, mm);
    m->mm_ws_bytes = mm;
    A((void**)&P.tok, (size_t)Mc * 4);
    A((void**)&P.X, (size_t)Mc * c.hidden * 4);
    A((void**)&P.Q, (size_t)Mc * qd * 4);
    A((void**)&P.K, (size_t)Mc * kvd * 4);
    A((void**)&P.V, (size_t)Mc * kvd * 4);
    A((void**)&P.A, (size_t)Mc * qd * 4);
    A((void**)&P.G, (size_t)Mc * c.ffn * 4);
    A((void**)&P.U, (size_t)Mc * c.ffn * 4);
    A((void**)&P.xn, (size_t)Mp * maxc * 4);
    A((void**)&P.xa, hexmm_xa_bytes(Mc, maxc, 1));
    A((void**)&P.xs, (size_t)Mp * 4);
    A((void**)&P.tmp, (size_t)kMaxSeg * Mc * kMaxRank * 4);
    A((void**)&P.part, part);
    return rc;
}

// One batched projection of the prepared operands (launch_batch_prep) into Y
// [M][rows]: y, or Y += y with accumulate.
int issue_mm(gsdh_model* m, const HexDev& t, int M, int cols, const float* tmp, float* Y, bool accumulate) {
    auto& P = m->pf;
    MatmulArgs a{};
    fill_seg(a.w, t, m, nullptr);
    const MatmulPlan plan = hexmm_plan(M, t.rows, cols, true);
    if (plan.nsplit > 1 && split_part_bytes(M, t.rows, cols) > P.part_bytes)
        return fail(-1, "prefill: split partials of %d tokens exceed the workspace", M);
    a.xa = P.xa; a.xs = P.xs; a.Xf = P.xn; a.hl = 1; a.accumulate = accumulate ? 1 : 0;
    a.tmp_k = t.k > 0 ? tmp : nullptr; a.Y = Y; a.M = M; a.cols = cols;
    a.nsplit = plan.nsplit; a.tg = plan.tg; a.rbw = plan.rbw; a.part = plan.nsplit > 1 ? P.part : nullptr;
    HIPCHK(launch_hexmm_prepared(a, m->stream));
    return 0;
}

// Operands of the batched projections reading X [M][cols] (norm: RMSNorm
// weights or null), with the rank-k projections of tensors t[0..n).
int issue_prep(gsdh_model* m, const float* X, int M, int cols, const float* norm_w, const HexDev* const* t, int n) {
    auto& P = m->pf;
    BatchPrep b{};
    b.X = X; b.ldx = cols; b.norm_w = norm_w; b.eps = m->c.rms_eps; b.M = M; b.cols = cols;
    b.xa = P.xa; b.xs = P.xs; b.xn = P.xn;
    for (int g = 0; g < n; g++) {
        if (t[g]->k > 0) {
            b.Vt[g] = t[g]->Vt; b.S[g] = t[g]->Sv; b.k[g] = t[g]->k;
            b.tmp[g] = P.tmp + (size_t)g * P.chunk * kMaxRank;
        }
    }
    HIPCHK(launch_batch_prep(b, m->stream));
    return 0;
}

// Prompt tokens P.tok[0..M) at positions p0.. through every layer as batched
// projections on the matrix cores (run_gpu_native_chat.py:892-956 per
// token, computed for M tokens at once), K/V appended for every position,
// causal attention over the cache; the last token's hidden state is left in
// x for the head.
int issue_prefill(gsdh_model* m, int M, int p0) {
    const auto& c = m->c;
    auto& P = m->pf;
    const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    int rc = 0;
    HIPCHK(launch_embed_rows(m->embed, P.tok, M, P.X, c.hidden, m->stream));
    for (int l = 0; l < c.n_layers; l++) {
        const HexDev *tq = &m->slot(l, GSDH_Q), *tk = &m->slot(l, GSDH_K), *tv = &m->slot(l, GSDH_V);
        const HexDev *to = &m->slot(l, GSDH_O), *tg = &m->slot(l, GSDH_GATE), *tu = &m->slot(l, GSDH_UP);
        const HexDev* td = &m->slot(l, GSDH_DOWN);
        const float* tmp0 = P.tmp;
        const float* tmp1 = P.tmp + (size_t)P.chunk * kMaxRank;
        const float* tmp2 = P.tmp + (size_t)2 * P.chunk * kMaxRank;
        {   // q, k, v of rmsnorm(x) * attn_norm
            const HexDev* ts[3] = {tq, tk, tv};
            if ((rc = issue_prep(m, P.X, M, c.hidden, m->norm(l, 0), ts, 3))) return rc;
            if ((rc = issue_mm(m, *tq, M, c.hidden, tmp0, P.Q, false))) return rc;
            if ((rc = issue_mm(m, *tk, M, c.hidden, tmp1, P.K, false))) return rc;
            if ((rc = issue_mm(m, *tv, M, c.hidden, tmp2, P.V, false))) return rc;
        }
        RopeKV r{};
        r.cs = m->cs; r.pos_dev = nullptr; r.pos = p0; r.k_cache = m->kc; r.v_cache = m->vc; r.layer = l;
        r.n_heads = c.n_heads; r.n_kv = c.n_kv_heads; r.hd = c.head_dim; r.max_seq = c.max_seq_len;
        r.interleaved = c.rope_interleaved;
        HIPCHK(launch_rope_kv_rows(P.Q, P.K, P.V, r, M, m->stream));
        {   // causal attention of the M tokens over the cache (matrix cores)
            PrefillAttn a{};
            a.q = P.Q; a.k_cache = m->kc; a.v_cache = m->vc; a.out = P.A; a.layer = l; a.p0 = p0; a.M = M;
            a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.hd = c.head_dim; a.max_seq = c.max_seq_len;
            a.sm_scale = 1.0f / (float)std::sqrt((double)c.head_dim);
            HIPCHK(launch_prefill_attention(a, m->stream));
        }
        {   // x += W_o attn
            const HexDev* ts[1] = {to};
            if ((rc = issue_prep(m, P.A, M, qd, nullptr, ts, 1))) return rc;
            if ((rc = issue_mm(m, *to, M, qd, tmp0, P.X, true))) return rc;
        }
        {   // h = silu(W_gate x') * (W_up x'), x' = rmsnorm(x) * ffn_norm
            const HexDev* ts[2] = {tg, tu};
            if ((rc = issue_prep(m, P.X, M, c.hidden, m->norm(l, 1), ts, 2))) return rc;
            if ((rc = issue_mm(m, *tg, M, c.hidden, tmp0, P.G, false))) return rc;
            if ((rc = issue_mm(m, *tu, M, c.hidden, tmp1, P.U, false))) return rc;
            HIPCHK(launch_swiglu(P.G, P.U, P.G, M * c.ffn, m->stream));
        }
        {   // x += W_down h
            const HexDev* ts[1] = {td};
            if ((rc = issue_prep(m, P.G, M, c.ffn, nullptr, ts, 1))) return rc;
            if ((rc = issue_mm(m, *td, M, c.ffn, tmp0, P.X, true))) return rc;
        }
    }
    (void)kvd;
    // the last token's residual stream for the head
    HIPCHK(hipMemcpyAsync(m->x, P.X + (size_t)(M - 1) * c.hidden, (size_t)c.hidden * 4, hipMemcpyDeviceToDevice,
                          m->stream));
    return 0;
}

// Prompt prompt[0..n) at positions start.. in batches of the prefill chunk;
// with `head`, the last token's logits and the greedy step (the step state
// then holds the first generated token at position start + n, gen_count 1).
// tok_stage: pinned host staging of n token ids (read by the copies until
// the stream is synchronised).  The step state's error word is cleared
// first and then only ever set, so a bounded wait that ran out in any
// chunk's attention reaches the caller.
int run_prefill(gsdh_model* m, const int* prompt, int n, int start, bool head, int* tok_stage) {
    auto& P = m->pf;
    HIPCHK(launch_set_step(m->st, prompt[0], start, 1, m->stream));
    for (int b0 = 0; b0 < n; b0 += P.chunk) {
        const int M = std::min(P.chunk, n - b0);
        int* ts = tok_stage + b0;
        for (int i = 0; i < M; i++) ts[i] = prompt[b0 + i];
        HIPCHK(hipMemcpyAsync(P.tok, ts, (size_t)M * 4, hipMemcpyHostToDevice, m->stream));
        int rc = issue_prefill(m, M, start + b0);
        if (rc) return rc;
    }
    HIPCHK(launch_set_step(m->st, prompt[n - 1], start + n - 1, 0, m->stream));
    if (head) return issue_head(m, true);
    return 0;
}

int capture(gsdh_model* m, bool with_head, int short_chunk, hipGraphExec_t* out) {
    hipGraph_t g = nullptr;
    HIPCHK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    int rc = issue_token(m, with_head, short_chunk);
    hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return fail((int)e, "hipStreamEndCapture: %s", hipGetErrorString(e));
    e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return fail((int)e, "hipGraphInstantiate: %s", hipGetErrorString(e));
    return 0;
}

}  // namespace

extern "C" {

int gsdh_model_create(const gsdh_model_config* cfg, gsdh_model** out) {
    if (!cfg || !out) return fail(-1, "model_create: null argument");
    const gsdh_model_config& c = *cfg;
    if (c.n_layers <= 0 || c.hidden <= 0 || c.ffn <= 0 || c.vocab <= 0 || c.max_seq_len <= 0)
        return fail(-1, "model_create: non-positive dimension");
    if (c.hidden % 64 || c.ffn % 64 || (c.n_heads * c.head_dim) % 64)
        return fail(-1, "model_create: hidden %d, ffn %d and n_heads*head_dim must be multiples of 64", c.hidden, c.ffn);
    if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256)
        return fail(-1, "model_create: head_dim %d not in {64,128,256}", c.head_dim);
    if (c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads || (8 % (c.n_heads / c.n_kv_heads)) != 0)
        return fail(-1, "model_create: n_heads %d / n_kv_heads %d is not a group size in {1,2,4,8}", c.n_heads, c.n_kv_heads);
    if (c.hidden > 65536 || c.ffn > 65536) return fail(-1, "model_create: dimension > 65536");
    gsdh_model* m = new gsdh_model();
    m->c = c;
    m->hex.resize((size_t)c.n_layers * 7 + 1);
    int rc = 0;
    auto A = [&](void** p, size_t n) { if (!rc) rc = dalloc(m, p, n); };
    hipError_t e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking);
    if (e != hipSuccess) { delete m; return fail((int)e, "hipStreamCreate: %s", hipGetErrorString(e)); }
    const size_t qd = (size_t)c.n_heads * c.head_dim, kvd = (size_t)c.n_kv_heads * c.head_dim;
    A((void**)&m->x, c.hidden * 4);
    A((void**)&m->q, qd * 4);
    A((void**)&m->k, kvd * 4);
    A((void**)&m->v, kvd * 4);
    A((void**)&m->attn, qd * 4);
    A((void**)&m->h, (size_t)c.ffn * 4);
    A((void**)&m->logits, (size_t)c.vocab * 4);
    const size_t kvn = (size_t)c.n_layers * c.max_seq_len * kvd;
    A((void**)&m->kc, kvn * 2);
    A((void**)&m->vc, kvn * 2);
    A((void**)&m->norms, ((size_t)c.n_layers * 2 + 1) * c.hidden * 4);
    A((void**)&m->embed, (size_t)c.vocab * c.hidden * 2);
    A((void**)&m->cs, (size_t)c.max_seq_len * (c.head_dim / 2) * sizeof(float2));
    m->chunk = attention_chunk(c.max_seq_len, c.n_kv_heads);
    m->max_splits = (c.max_seq_len + m->chunk - 1) / m->chunk;
    A((void**)&m->ws, attention_ws_bytes(c.n_kv_heads, m->max_splits, c.n_heads / c.n_kv_heads, c.head_dim));
    A((void**)&m->counters, (size_t)c.n_kv_heads * 4);
    m->pub_words = (4 * c.n_layers + 1) * kLeadMax;
    A((void**)&m->pub, (size_t)m->pub_words * 8);
    A((void**)&m->fa_words, (qd + kvd) * 8);
    A((void**)&m->fa_epoch, 4);
    A((void**)&m->am_words, 3 * kArgBlocks * 8);
    A((void**)&m->am_ctr, kArgBlocks * 4);
    {
        const char* fe = std::getenv("GSD_FUSED_ATTN");
        m->fa_on = !(fe && fe[0] == '0');
        fe = std::getenv("GSD_FUSED_FFN");
        m->ffn_on = !(fe && fe[0] == '0') && ffn_supported(c.hidden, c.ffn);
        fe = std::getenv("GSD_FUSED_OFFN");
        m->offn_on = m->ffn_on && !(fe && fe[0] == '0') && c.n_heads * c.head_dim == c.hidden;
    }
    if (m->ffn_on) {
        A((void**)&m->ffn_words, ffn_words(c.hidden, c.ffn) * 8);
        A((void**)&m->ffn_ctr, kFfnMaxGrid * 4);
    }
    A((void**)&m->st, sizeof(StepState));
    A((void**)&m->gen_tok, (size_t)c.max_seq_len * 4);
    A((void**)&m->gen_margin, (size_t)c.max_seq_len * 4);
    for (int R = 1; R <= 8; R++) {
        std::vector<float> t = host_table(R);
        A((void**)&m->tables[R], t.size() * 4);
        if (!rc) {
            e = hipMemcpy(m->tables[R], t.data(), t.size() * 4, hipMemcpyHostToDevice);
            if (e != hipSuccess) rc = fail((int)e, "hipMemcpy table: %s", hipGetErrorString(e));
        }
        std::vector<uint32_t> f = host_fields(R);
        f.resize(kTableSlots, 0u);   // padded: the matvec reads 16-entry slices
        A((void**)&m->fields[R], f.size() * 4);
        if (!rc) {
            e = hipMemcpy(m->fields[R], f.data(), f.size() * 4, hipMemcpyHostToDevice);
            if (e != hipSuccess) rc = fail((int)e, "hipMemcpy fields: %s", hipGetErrorString(e));
        }
    }
    if (!rc) {
        e = hipHostMalloc((void**)&m->st_host, sizeof(StepState) * 2, 0);
        if (e != hipSuccess) rc = fail((int)e, "hipHostMalloc: %s", hipGetErrorString(e));
    }
    if (!rc) {
        // zero the KV cache and counters with kernels (no memset nodes anywhere)
        e = launch_fill_u32(m->counters, 0u, (size_t)c.n_kv_heads, m->stream);
        if (e == hipSuccess)
            e = launch_fill_u32(reinterpret_cast<unsigned*>(m->ws), 0u,
                                attention_ws_bytes(c.n_kv_heads, m->max_splits, c.n_heads / c.n_kv_heads, c.head_dim) / 4,
                                m->stream);
        if (e == hipSuccess) e = launch_fill_u32((unsigned*)m->pub, 0u, 2 * (size_t)m->pub_words, m->stream);
        if (e == hipSuccess) e = launch_fill_u32((unsigned*)m->fa_words, 0u, 2 * (qd + kvd), m->stream);
        if (e == hipSuccess) e = launch_fill_u32(m->fa_epoch, 0u, 1, m->stream);
        if (e == hipSuccess) e = launch_fill_u32((unsigned*)m->am_words, 0u, 6 * kArgBlocks, m->stream);
        if (e == hipSuccess) e = launch_fill_u32(m->am_ctr, 0u, kArgBlocks, m->stream);
        if (e == hipSuccess && m->ffn_on)
            e = launch_fill_u32((unsigned*)m->ffn_words, 0u, 2 * ffn_words(c.hidden, c.ffn), m->stream);
        if (e == hipSuccess && m->ffn_on) e = launch_fill_u32(m->ffn_ctr, 0u, kFfnMaxGrid, m->stream);
        if (e == hipSuccess) e = launch_fill_u32((unsigned*)m->kc, 0u, kvn / 2, m->stream);
        if (e == hipSuccess) e = launch_fill_u32((unsigned*)m->vc, 0u, kvn / 2, m->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
        if (e != hipSuccess) rc = fail((int)e, "model init: %s", hipGetErrorString(e));
    }
    if (!rc) {
        // RoPE table [pos][i] = (cos, sin), evaluated like the reference engine
        std::vector<float> cs((size_t)c.max_seq_len * c.head_dim);
        for (int p = 0; p < c.max_seq_len; p++) rope_cs(c.rope_theta, c.head_dim, p, cs.data() + (size_t)p * c.head_dim);
        e = hipMemcpy(m->cs, cs.data(), cs.size() * 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) rc = fail((int)e, "hipMemcpy rope: %s", hipGetErrorString(e));
    }
    if (rc) {
        gsdh_model_destroy(m);
        return rc;
    }
    *out = m;
    return 0;
}

int gsdh_model_destroy(gsdh_model* m) {
    if (!m) return 0;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    for (hipGraphExec_t g : {m->g_full, m->g_prefill})
        if (g) (void)hipGraphExecDestroy(g);
    for (int t = 0; t < kShortTiers; t++)
        for (hipGraphExec_t g : {m->g_full_s[t], m->g_prefill_s[t]})
            if (g) (void)hipGraphExecDestroy(g);
    for (auto& t : m->hex)
        if (t.block) (void)hipFree(t.block);
    for (void* p : m->allocs) (void)hipFree(p);
    if (m->st_host) (void)hipHostFree(m->st_host);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
    return 0;
}

int gsdh_model_set_embedding(gsdh_model* m, const uint16_t* embed) {
    if (m->finalized) return fail(-1, "set_embedding: the model is finalized (its token graphs hold the tensors)");
    HIPCHK(hipMemcpy(m->embed, embed, (size_t)m->c.vocab * m->c.hidden * 2, hipMemcpyHostToDevice));
    return 0;
}

int gsdh_model_set_norm(gsdh_model* m, int layer, int which, const float* w) {
    if (m->finalized) return fail(-1, "set_norm: the model is finalized (its token graphs hold the tensors)");
    if (layer >= m->c.n_layers || which < 0 || which > 1) return fail(-1, "set_norm: layer %d which %d", layer, which);
    HIPCHK(hipMemcpy(m->norm(layer, which), w, (size_t)m->c.hidden * 4, hipMemcpyHostToDevice));
    return 0;
}

int gsdh_model_set_hex(gsdh_model* m, int layer, int slot, int radius, int rows, int cols, int k_dim,
                       const uint8_t* codes, const uint16_t* scales, const uint32_t* row_ptr,
                       const uint16_t* kink_cols, const float* kink_deltas, int64_t nk, const uint16_t* U,
                       const float* Sv, const uint16_t* Vt) {
    const auto& c = m->c;
    if (m->finalized) return fail(-1, "set_hex: the model is finalized (its token graphs hold the tensors)");
    if (slot < 0 || slot > GSDH_LM_HEAD) return fail(-1, "set_hex: slot %d", slot);
    if (slot != GSDH_LM_HEAD && (layer < 0 || layer >= c.n_layers)) return fail(-1, "set_hex: layer %d", layer);
    const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    int er = 0, ec = 0;
    switch (slot) {
        case GSDH_Q: er = qd; ec = c.hidden; break;
        case GSDH_K: case GSDH_V: er = kvd; ec = c.hidden; break;
        case GSDH_O: er = c.hidden; ec = qd; break;
        case GSDH_GATE: case GSDH_UP: er = c.ffn; ec = c.hidden; break;
        case GSDH_DOWN: er = c.hidden; ec = c.ffn; break;
        default: er = c.vocab; ec = c.hidden; break;
    }
    if (rows != er || cols != ec) return fail(-1, "set_hex: layer %d slot %d shape %dx%d, expected %dx%d", layer, slot, rows, cols, er, ec);
    if (radius < 1 || radius > 8) return fail(-1, "set_hex: radius %d outside 1..8", radius);
    if (k_dim < 0 || k_dim > kMaxRank) return fail(-1, "set_hex: k_dim %d outside 0..%d", k_dim, kMaxRank);
    if (k_dim > 0 && (!U || !Sv || !Vt)) return fail(-1, "set_hex: k_dim %d without U/S/Vt", k_dim);
    if (nk < 0 || (nk > 0 && (!kink_cols || !kink_deltas))) return fail(-1, "set_hex: nk %lld", (long long)nk);
    const int n_pts = 3 * radius * radius + 3 * radius + 1;
    const size_t ncodes = (size_t)rows * cols / 2;
    // validate: codes < n_pts, CSR monotone and ending at nk, kink columns < cols
    for (size_t i = 0; i < ncodes; i++)
        if (codes[i] >= n_pts) return fail(-1, "set_hex: code %u at %zu >= n_pts %d (layer %d slot %d)", codes[i], i, n_pts, layer, slot);
    if (row_ptr[0] != 0) return fail(-1, "set_hex: row_ptr[0] != 0");
    for (int r = 0; r < rows; r++)
        if (row_ptr[r + 1] < row_ptr[r]) return fail(-1, "set_hex: row_ptr not monotone at row %d", r);
    if ((int64_t)row_ptr[rows] != nk) return fail(-1, "set_hex: row_ptr[rows]=%u but %lld kinks", row_ptr[rows], (long long)nk);
    for (int64_t i = 0; i < nk; i++)
        if (kink_cols[i] >= cols) return fail(-1, "set_hex: kink column %u >= cols %d", kink_cols[i], cols);

    HexDev& t = m->slot(layer, slot);
    if (t.block) { (void)hipFree(t.block); m->dev_bytes -= t.bytes; t = HexDev(); }
    auto al = [](size_t n) { return (n + 255) / 256 * 256; };
    // tiled layout of the MFMA matvec: codes [nrb][nc][tile] where lane l of
    // a tile holds 16 codes of row 16rb + (l & 15): code j = pair 64c +
    // 8(l >> 4) + j (j < 8) or 64c + 32 + 8(l >> 4) + j - 8 (j >= 8).  A tile
    // is 64 lanes x 16 bytes (one byte per code) for codebooks of more than
    // 128 points, and 896 bytes for at most 128 (radius <= 6): 7 bits per
    // code, lane pair i at bytes 28i .. 28i + 27, lane 2i's 16 codes as a
    // 112-bit little-endian field at byte 28i (code j = bits 7j .. 7j + 6),
    // lane 2i + 1's at byte 28i + 14.  Scales [nrb][nc][16] as the fp16 pair
    // of the chunk's two 64-weight blocks.  Padding: code 0, scale 0.
    const size_t nrb = ((size_t)rows + 15) / 16, nc = ((size_t)cols + 127) / 128, nsb = (size_t)cols / 64;
    const size_t half = (size_t)cols / 2;
    const bool b7 = n_pts <= 128;
    const size_t tbytes = b7 ? 896 : 1024;
    const size_t o_codes = 0, o_sc = o_codes + al(nrb * nc * tbytes), o_rp = o_sc + al(nrb * nc * 64);
    const size_t o_kc = o_rp + al((size_t)(rows + 1) * 4), o_kd = o_kc + al((size_t)nk * 2);
    const size_t o_u = o_kd + al((size_t)nk * 4), o_s = o_u + al((size_t)rows * k_dim * 2);
    const size_t o_vt = o_s + al((size_t)k_dim * 4), o_end = o_vt + al((size_t)k_dim * cols * 2);
    // down of a model the fused FFN launch covers: also its column slabs
    // (FfnArgs::dcodes): slab b = columns 64 b .. 64 b + 63, step sd = rows
    // 32 sd .. 32 sd + 31, lane l: row 32 sd + (l & 15) in codes 0-7 and row
    // 32 sd + 16 + (l & 15) in codes 8-15, pair 8 (l >> 4) + (j & 7) of the
    // slab; the scale word: those two rows' scales of block b
    const bool slabs = slot == GSDH_DOWN && m->ffn_on;
    const size_t nslab = (size_t)cols / 64, nsd = ((size_t)rows + 31) / 32;
    const size_t o_ds = o_end, o_dss = o_ds + (slabs ? al(nslab * nsd * tbytes) : 0);
    const size_t total = o_dss + (slabs ? al(nslab * nsd * 64) : 0);
    void* blk = nullptr;
    HIPCHK(hipMalloc(&blk, total));
    char* b = static_cast<char*>(blk);
    t.block = blk; t.bytes = total; m->dev_bytes += total;
    t.codes_t = (uint4*)(b + o_codes); t.scales_t = (uint32_t*)(b + o_sc); t.row_ptr = (uint32_t*)(b + o_rp);
    t.kcols = (uint16_t*)(b + o_kc); t.kdel = (float*)(b + o_kd); t.U = (uint16_t*)(b + o_u);
    t.Sv = (float*)(b + o_s); t.Vt = (uint16_t*)(b + o_vt);
    // lane l's code j (value v) into a tile at dst
    auto put_code = [b7](uint8_t* dst, int l, int j, unsigned v) {
        uint8_t* ld = b7 ? dst + 28 * (l >> 1) + 14 * (l & 1) : dst + 16 * l;
        if (!b7) {
            ld[j] = (uint8_t)v;
        } else {   // bits 7j .. 7j + 6 of the lane's field
            const unsigned bit = 7u * (unsigned)j;
            ld[bit >> 3] |= (uint8_t)(v << (bit & 7));
            if ((bit & 7) > 1) ld[(bit >> 3) + 1] |= (uint8_t)(v >> (8 - (bit & 7)));
        }
    };
    {
        std::vector<uint8_t> ct(nrb * nc * tbytes, 0);
        std::vector<uint32_t> stl(nrb * nc * 16, 0);
        for (size_t rb = 0; rb < nrb; rb++)
            for (size_t c = 0; c < nc; c++) {
                uint8_t* dst = ct.data() + (rb * nc + c) * tbytes;
                for (int l = 0; l < 64; l++) {
                    const size_t row = rb * 16 + (size_t)(l & 15);
                    if (row >= (size_t)rows) continue;
                    const uint8_t* src = codes + row * half;
                    for (int j = 0; j < 16; j++) {
                        const size_t p = 64 * c + (j < 8 ? 8 * (size_t)(l >> 4) + j : 32 + 8 * (size_t)(l >> 4) + (j - 8));
                        put_code(dst, l, j, p < half ? src[p] : 0u);
                    }
                }
                for (int n = 0; n < 16; n++) {
                    const size_t row = rb * 16 + (size_t)n;
                    if (row >= (size_t)rows) continue;
                    const uint32_t s0 = scales[row * nsb + 2 * c];
                    const uint32_t s1 = 2 * c + 1 < nsb ? scales[row * nsb + 2 * c + 1] : 0u;
                    stl[(rb * nc + c) * 16 + n] = s0 | (s1 << 16);
                }
            }
        HIPCHK(hipMemcpy(t.codes_t, ct.data(), ct.size(), hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(t.scales_t, stl.data(), stl.size() * 4, hipMemcpyHostToDevice));
    }
    if (slabs) {
        t.dslab = (unsigned char*)(b + o_ds);
        t.dslab_sc = (uint32_t*)(b + o_dss);
        std::vector<uint8_t> ct(nslab * nsd * tbytes, 0);
        std::vector<uint32_t> stl(nslab * nsd * 16, 0);
        for (size_t sb = 0; sb < nslab; sb++)
            for (size_t sd = 0; sd < nsd; sd++) {
                const size_t ti = sb * nsd + sd;
                uint8_t* dst = ct.data() + ti * tbytes;
                for (int l = 0; l < 64; l++)
                    for (int j = 0; j < 16; j++) {
                        const size_t row = 32 * sd + 16 * (size_t)(j >> 3) + (size_t)(l & 15);
                        if (row >= (size_t)rows) continue;
                        put_code(dst, l, j, codes[row * half + 32 * sb + 8 * (size_t)(l >> 4) + (size_t)(j & 7)]);
                    }
                for (int n = 0; n < 16; n++) {
                    const size_t r0 = 32 * sd + (size_t)n, r1 = r0 + 16;
                    const uint32_t s0 = r0 < (size_t)rows ? scales[r0 * nsb + sb] : 0u;
                    const uint32_t s1 = r1 < (size_t)rows ? scales[r1 * nsb + sb] : 0u;
                    stl[ti * 16 + n] = s0 | (s1 << 16);
                }
            }
        HIPCHK(hipMemcpy(t.dslab, ct.data(), ct.size(), hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(t.dslab_sc, stl.data(), stl.size() * 4, hipMemcpyHostToDevice));
    }
    HIPCHK(hipMemcpy(t.row_ptr, row_ptr, (size_t)(rows + 1) * 4, hipMemcpyHostToDevice));
    if (nk > 0) {
        HIPCHK(hipMemcpy(t.kcols, kink_cols, (size_t)nk * 2, hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(t.kdel, kink_deltas, (size_t)nk * 4, hipMemcpyHostToDevice));
    }
    if (k_dim > 0) {
        HIPCHK(hipMemcpy(t.U, U, (size_t)rows * k_dim * 2, hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(t.Sv, Sv, (size_t)k_dim * 4, hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(t.Vt, Vt, (size_t)k_dim * cols * 2, hipMemcpyHostToDevice));
    }
    t.set = 1; t.radius = radius; t.rows = rows; t.cols = cols; t.k = k_dim; t.nk = nk;
    return 0;
}

int gsdh_model_finalize(gsdh_model* m) {
    for (int l = 0; l < m->c.n_layers; l++)
        for (int s = 0; s < 7; s++)
            if (!m->slot(l, s).set) return fail(-1, "finalize: layer %d slot %d not set", l, s);
    if (!m->slot(0, GSDH_LM_HEAD).set) return fail(-1, "finalize: lm_head not set");
    int rc = capture(m, true, 0, &m->g_full);
    if (!rc) rc = capture(m, false, 0, &m->g_prefill);
    for (int t = 0; t < kShortTiers && !rc; t++) {
        rc = capture(m, true, kShortChunk[t], &m->g_full_s[t]);
        if (!rc) rc = capture(m, false, kShortChunk[t], &m->g_prefill_s[t]);
    }
    if (!rc) rc = setup_batched(m);
    if (rc) return rc;
    HIPCHK(hipStreamSynchronize(m->stream));
    m->finalized = true;
    return 0;
}

uint64_t gsdh_model_device_bytes(gsdh_model* m) { return m ? m->dev_bytes : 0; }

int gsdh_forward_token(gsdh_model* m, int token_id, int pos, int want_logits, float* logits_host, int* argmax_out) {
    if (!m->finalized) return fail(-1, "forward_token: model not finalized");
    if (token_id < 0 || token_id >= m->c.vocab) return fail(-1, "forward_token: token %d outside vocab %d", token_id, m->c.vocab);
    if (pos < 0 || pos >= m->c.max_seq_len) return fail(-1, "forward_token: pos %d outside 0..%d", pos, m->c.max_seq_len - 1);
    StepState* h = m->st_host;
    *h = StepState{};
    h->token = token_id; h->pos = pos;
    HIPCHK(hipMemcpyAsync(m->st, h, sizeof(StepState), hipMemcpyHostToDevice, m->stream));
    HIPCHK(hipGraphLaunch(token_graph(m, want_logits != 0, pos), m->stream));
    if (want_logits && logits_host)
        HIPCHK(hipMemcpyAsync(logits_host, m->logits, (size_t)m->c.vocab * 4, hipMemcpyDeviceToHost, m->stream));
    HIPCHK(hipMemcpyAsync(m->st_host + 1, m->st, sizeof(StepState), hipMemcpyDeviceToHost, m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    if (m->st_host[1].err) return fail(-2, "forward_token: an in-kernel wait timed out");
    if (want_logits && argmax_out) *argmax_out = m->st_host[1].token;
    return 0;
}

int gsdh_generate_greedy(gsdh_model* m, const int* prompt, int n_prompt, int start_pos, int n_new, int* tokens_out,
                         float* margins_out) {
    if (!m->finalized) return fail(-1, "generate: model not finalized");
    if (n_prompt <= 0 || n_new <= 0) return fail(-1, "generate: n_prompt %d n_new %d", n_prompt, n_new);
    if (start_pos < 0 || start_pos + n_prompt + n_new - 1 > m->c.max_seq_len)
        return fail(-1, "generate: positions %d..%d exceed max_seq_len %d", start_pos, start_pos + n_prompt + n_new - 1, m->c.max_seq_len);
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= m->c.vocab) return fail(-1, "generate: prompt token %d outside vocab", prompt[i]);
    int* tok_stage = nullptr;
    HIPCHK(hipHostMalloc((void**)&tok_stage, sizeof(int) * (size_t)n_prompt, 0));
    int rc = 0;
    if (m->pf.batched) {
        rc = run_prefill(m, prompt, n_prompt, start_pos, true, tok_stage);
    } else {
        // token by token: the step state of each prompt token, its error
        // word cleared for the first only (a wait that ran out stays set)
        for (int i = 0; i < n_prompt && !rc; i++) {
            hipError_t e = launch_set_step(m->st, prompt[i], start_pos + i, i == 0 ? 1 : 0, m->stream);
            if (e == hipSuccess) e = hipGraphLaunch(token_graph(m, i == n_prompt - 1, start_pos + i), m->stream);
            if (e != hipSuccess) rc = fail((int)e, "generate prefill: %s", hipGetErrorString(e));
        }
    }
    for (int i = 1; i < n_new && !rc; i++) {
        // the device advances the position: this launch runs the token at
        // start_pos + n_prompt - 1 + i
        hipError_t e = hipGraphLaunch(token_graph(m, true, start_pos + n_prompt - 1 + i), m->stream);
        if (e != hipSuccess) rc = fail((int)e, "generate decode: %s", hipGetErrorString(e));
    }
    if (!rc) {
        hipError_t e = hipMemcpyAsync(tokens_out, m->gen_tok, (size_t)n_new * 4, hipMemcpyDeviceToHost, m->stream);
        if (e == hipSuccess && margins_out) e = hipMemcpyAsync(margins_out, m->gen_margin, (size_t)n_new * 4, hipMemcpyDeviceToHost, m->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(m->st_host + 1, m->st, sizeof(StepState), hipMemcpyDeviceToHost, m->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
        if (e != hipSuccess) rc = fail((int)e, "generate readback: %s", hipGetErrorString(e));
        else if (m->st_host[1].err) rc = fail(-2, "generate: an in-kernel wait timed out");
    }
    (void)hipStreamSynchronize(m->stream);
    (void)hipHostFree(tok_stage);
    return rc;
}

int gsdh_model_prefill(gsdh_model* m, const int* tokens, int n, int start_pos, int want_logits, float* logits_host,
                       int* argmax_out) {
    if (!m || !tokens) return fail(-1, "prefill: null argument");
    if (!m->finalized) return fail(-1, "prefill: model not finalized");
    if (n <= 0) return fail(-1, "prefill: n %d", n);
    if (start_pos < 0 || start_pos + n > m->c.max_seq_len)
        return fail(-1, "prefill: positions %d..%d exceed max_seq_len %d", start_pos, start_pos + n - 1, m->c.max_seq_len);
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->c.vocab) return fail(-1, "prefill: token %d outside vocab %d", tokens[i], m->c.vocab);
    StepState* ring = nullptr;
    HIPCHK(hipHostMalloc((void**)&ring, sizeof(StepState) * 2 + sizeof(int) * (size_t)n, 0));
    int rc = run_prefill(m, tokens, n, start_pos, want_logits != 0, reinterpret_cast<int*>(ring + 2));
    if (!rc && want_logits && logits_host) {
        hipError_t e = hipMemcpyAsync(logits_host, m->logits, (size_t)m->c.vocab * 4, hipMemcpyDeviceToHost, m->stream);
        if (e != hipSuccess) rc = fail((int)e, "prefill: %s", hipGetErrorString(e));
    }
    if (!rc) {
        hipError_t e = hipMemcpyAsync(ring + 1, m->st, sizeof(StepState), hipMemcpyDeviceToHost, m->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
        if (e != hipSuccess) rc = fail((int)e, "prefill: %s", hipGetErrorString(e));
        else if (ring[1].err) rc = fail(-2, "prefill: an in-kernel wait timed out");
        else if (want_logits && argmax_out) *argmax_out = ring[1].token;
    }
    (void)hipStreamSynchronize(m->stream);
    (void)hipHostFree(ring);
    return rc;
}

int gsdh_model_fused_ffn(gsdh_model* m, int layer) {
    if (!m) return fail(-1, "fused_ffn: null model");
    if (layer < 0 || layer >= m->c.n_layers) return fail(-1, "fused_ffn: layer %d", layer);
    return ffn_fused(m, layer) ? (offn_fused(m, layer) ? 2 : 1) : 0;
}

int gsdh_model_set_prefill(gsdh_model* m, int batched) {
    if (!m) return fail(-1, "set_prefill: null model");
    m->pf.batched = batched != 0;
    return 0;
}

int gsdh_model_read_codes(gsdh_model* m, int layer, int slot, uint8_t* codes_out) {
    if (!m || !codes_out) return fail(-1, "read_codes: null argument");
    if (slot < 0 || slot > GSDH_LM_HEAD) return fail(-1, "read_codes: slot %d", slot);
    if (slot != GSDH_LM_HEAD && (layer < 0 || layer >= m->c.n_layers)) return fail(-1, "read_codes: layer %d", layer);
    const HexDev& t = m->slot(layer, slot);
    if (!t.set) return fail(-1, "read_codes: layer %d slot %d not set", layer, slot);
    const size_t n = (size_t)t.rows * t.cols / 2;
    void* d = nullptr;
    HIPCHK(hipMalloc(&d, n));
    HexSeg s{};
    fill_seg(s, t, m, nullptr);
    hipError_t e = launch_tile_codes(s, t.cols, static_cast<uint8_t*>(d), m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    if (e == hipSuccess) e = hipMemcpy(codes_out, d, n, hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (e != hipSuccess) return fail((int)e, "read_codes: %s", hipGetErrorString(e));
    return 0;
}

int gsdh_model_matmul(gsdh_model* m, int layer, int slot, const uint16_t* X, int M, float* Y) {
    return gsdh_model_matmul_shared(m, layer, &slot, 1, X, M, &Y);
}

int gsdh_model_matmul_shared(gsdh_model* m, int layer, const int* slots, int n, const uint16_t* X, int M,
                             float* const* Y) {
    if (!m || !X || !slots || !Y) return fail(-1, "matmul: null argument");
    if (n < 1 || n > kMaxSeg) return fail(-1, "matmul: %d tensors (1..%d share one input)", n, kMaxSeg);
    if (M <= 0) return fail(-1, "matmul: M %d", M);
    if (!m->finalized) return fail(-1, "matmul: model not finalized");
    if (M > kMatmulMaxM) return fail(-1, "matmul: M %d > %d tokens per call (split the batch)", M, kMatmulMaxM);
    const HexDev* ts[kMaxSeg] = {};
    for (int i = 0; i < n; i++) {
        const int slot = slots[i];
        if (slot < 0 || slot > GSDH_LM_HEAD) return fail(-1, "matmul: slot %d", slot);
        if (slot != GSDH_LM_HEAD && (layer < 0 || layer >= m->c.n_layers)) return fail(-1, "matmul: layer %d", layer);
        if (!Y[i]) return fail(-1, "matmul: null output %d", i);
        ts[i] = &m->slot(layer, slot);
        if (!ts[i]->set) return fail(-1, "matmul: layer %d slot %d not set", layer, slot);
        if (ts[i]->cols != ts[0]->cols) return fail(-1, "matmul: tensors of %d and %d columns do not share an input",
                                                    ts[0]->cols, ts[i]->cols);
        if (matmul_ws_need(M, ts[i]->rows, ts[i]->cols) > m->mm_ws_bytes)
            return fail(-1, "matmul: staging for %d tokens exceeds the model's workspace", M);
    }
    const int cols = ts[0]->cols;
    const size_t xa = (hexmm_xa_bytes(M, cols) + 255) / 256 * 256;
    const size_t xs = ((size_t)(M + 15) / 16 * 16 * 4 + 255) / 256 * 256;
    const size_t tk = ((size_t)M * kMaxRank * 4 + 255) / 256 * 256;
    char* w = static_cast<char*>(m->mm_ws);
    // X's operands once for every tensor of the call
    HIPCHK(launch_hexmm_xprep(X, M, cols, reinterpret_cast<uint4*>(w), reinterpret_cast<float*>(w + xa), m->stream));
    for (int i = 0; i < n; i++) {
        const HexDev& t = *ts[i];
        const MatmulPlan plan = hexmm_plan(M, t.rows, t.cols);
        float* tmp = reinterpret_cast<float*>(w + xa + xs + (size_t)i * tk);
        MatmulArgs a{};
        fill_seg(a.w, t, m, nullptr);
        a.X = X;
        a.xa = reinterpret_cast<uint4*>(w);
        a.xs = reinterpret_cast<float*>(w + xa);
        a.tmp_k = t.k > 0 ? tmp : nullptr;
        a.Y = Y[i];
        a.M = M;
        a.cols = t.cols;
        a.nsplit = plan.nsplit;
        a.tg = plan.tg;
        a.rbw = plan.rbw;
        a.prepped = 1;
        // (split partials of the tensors in turn: stream order keeps them apart)
        a.part = plan.nsplit > 1 ? reinterpret_cast<float*>(w + xa + xs + kMaxSeg * tk) : nullptr;
        if (t.k > 0) HIPCHK(launch_lowrank_batched(X, t.Vt, t.Sv, tmp, M, t.k, t.cols, m->stream));
        HIPCHK(launch_hexmm(a, m->stream));
    }
    return 0;
}

int gsdh_matmul_plan(int M, int rows, int cols, int* tg, int* rbw, int* nsplit) {
    if (M <= 0 || rows <= 0 || cols <= 0 || !tg || !rbw || !nsplit) return fail(-1, "matmul_plan: bad argument");
    const MatmulPlan p = hexmm_plan(M, rows, cols);
    *tg = p.tg;
    *rbw = p.rbw;
    *nsplit = p.nsplit;
    return 0;
}

int gsdh_model_run_linear(gsdh_model* m, int layer, int mask) {
    if (!m) return fail(-1, "run_linear: null model");
    if (mask & ~31) return fail(-1, "run_linear: mask 0x%x", mask);
    if (mask == 16) {   // the head alone: final norm + lm_head, no argmax
        const bool publish = m->slot(0, GSDH_LM_HEAD).k > 2;
        m->pub_next = 0;
        if (publish) HIPCHK(launch_fill_u32((unsigned*)m->pub, 0u, 2 * (size_t)kLeadMax, m->stream));
        return issue_head(m, false);
    }
    if (mask & 16) return fail(-1, "run_linear: the head (mask 16) runs alone");
    if (layer < 0 || layer >= m->c.n_layers) return fail(-1, "run_linear: layer %d", layer);
    // a sequence of its own: its publication words (only launches with a rank
    // above 2 publish their projections; smaller ranks are formed in every
    // block) start at zero
    static const int slots[4][2] = {{GSDH_Q, GSDH_V}, {GSDH_O, GSDH_O}, {GSDH_GATE, GSDH_UP}, {GSDH_DOWN, GSDH_DOWN}};
    bool publish = false;
    for (int i = 0; i < 4; i++)
        if (mask & (1 << i))
            for (int s = slots[i][0]; s <= slots[i][1]; s++) publish = publish || m->slot(layer, s).k > 2;
    m->pub_next = 0;
    if (publish) HIPCHK(launch_fill_u32((unsigned*)m->pub, 0u, 2 * (size_t)4 * kLeadMax, m->stream));
    return issue_linear(m, layer, mask);
}

int gsdh_model_capture_begin(gsdh_model* m) {
    HIPCHK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    return 0;
}

int gsdh_model_capture_end(gsdh_model* m, void** graph_exec_out) {
    hipGraph_t g = nullptr;
    HIPCHK(hipStreamEndCapture(m->stream, &g));
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return fail((int)e, "hipGraphInstantiate: %s", hipGetErrorString(e));
    *graph_exec_out = ge;
    return 0;
}

int gsdh_graph_launch(gsdh_model* m, void* ge, int n) {
    for (int i = 0; i < n; i++) HIPCHK(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(ge), m->stream));
    return 0;
}

int gsdh_graph_time(gsdh_model* m, void* ge, int n, float* ms_out) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    HIPCHK(hipEventCreate(&e0));
    hipError_t e = hipEventCreate(&e1);
    if (e != hipSuccess) { (void)hipEventDestroy(e0); return fail((int)e, "hipEventCreate: %s", hipGetErrorString(e)); }
    e = hipEventRecord(e0, m->stream);
    for (int i = 0; i < n && e == hipSuccess; i++) e = hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(ge), m->stream);
    if (e == hipSuccess) e = hipEventRecord(e1, m->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (e != hipSuccess) return fail((int)e, "graph_time: %s", hipGetErrorString(e));
    *ms_out = ms;
    return 0;
}

int gsdh_graph_destroy(void* ge) {
    HIPCHK(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(ge)));
    return 0;
}

void* gsdh_model_stream(gsdh_model* m) { return m ? (void*)m->stream : nullptr; }

int gsdh_model_vector(gsdh_model* m, int which, int write, void* host, uint64_t nbytes) {
    if (!m || !host) return fail(-1, "model_vector: null argument");
    const auto& c = m->c;
    float* d = nullptr;
    size_t n = 0;
    switch (which) {
        case GSDH_VEC_X: d = m->x; n = c.hidden; break;
        case GSDH_VEC_Q: d = m->q; n = (size_t)c.n_heads * c.head_dim; break;
        case GSDH_VEC_K: d = m->k; n = (size_t)c.n_kv_heads * c.head_dim; break;
        case GSDH_VEC_V: d = m->v; n = (size_t)c.n_kv_heads * c.head_dim; break;
        case GSDH_VEC_ATTN: d = m->attn; n = (size_t)c.n_heads * c.head_dim; break;
        case GSDH_VEC_H: d = m->h; n = c.ffn; break;
        case GSDH_VEC_LOGITS: d = m->logits; n = c.vocab; break;
        default: return fail(-1, "model_vector: unknown vector %d", which);
    }
    if (nbytes != n * 4) return fail(-1, "model_vector: %llu bytes, vector %d holds %zu", (unsigned long long)nbytes, which, n * 4);
    HIPCHK(hipStreamSynchronize(m->stream));
    HIPCHK(hipMemcpy(write ? (void*)d : host, write ? host : (const void*)d, nbytes,
                     write ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost));
    return 0;
}

int gsdh_model_set_step(gsdh_model* m, int token_id, int pos) {
    if (!m) return fail(-1, "set_step: null model");
    if (token_id < 0 || token_id >= m->c.vocab) return fail(-1, "set_step: token %d outside vocab %d", token_id, m->c.vocab);
    if (pos < 0 || pos >= m->c.max_seq_len) return fail(-1, "set_step: pos %d outside 0..%d", pos, m->c.max_seq_len - 1);
    HIPCHK(hipStreamSynchronize(m->stream));
    StepState* h = m->st_host;
    *h = StepState{};
    h->token = token_id; h->pos = pos;
    HIPCHK(hipMemcpy(m->st, h, sizeof(StepState), hipMemcpyHostToDevice));
    return 0;
}

int gsdh_model_read_kv(gsdh_model* m, int layer, int pos, uint16_t* k_out, uint16_t* v_out) {
    if (!m || !k_out || !v_out) return fail(-1, "read_kv: null argument");
    const auto& c = m->c;
    if (layer < 0 || layer >= c.n_layers) return fail(-1, "read_kv: layer %d", layer);
    if (pos < 0 || pos >= c.max_seq_len) return fail(-1, "read_kv: pos %d outside 0..%d", pos, c.max_seq_len - 1);
    const size_t kvd = (size_t)c.n_kv_heads * c.head_dim, off = ((size_t)layer * c.max_seq_len + pos) * kvd;
    HIPCHK(hipStreamSynchronize(m->stream));
    HIPCHK(hipMemcpy(k_out, m->kc + off, kvd * 2, hipMemcpyDeviceToHost));
    HIPCHK(hipMemcpy(v_out, m->vc + off, kvd * 2, hipMemcpyDeviceToHost));
    return 0;
}

}  // extern "C"
