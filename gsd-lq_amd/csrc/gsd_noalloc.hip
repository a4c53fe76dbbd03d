// gsd_noalloc.hip -- gsdh_gqa_attention_noalloc: the decode attention twin for
// callers that cannot allocate device memory (HIP graph capture, serving
// loops, harnesses that forbid hipMalloc).  Its split partials live in a
// file-scope device array.  The operator twins gsdh_gqa_attention and
// gsdh_rope_store_gqa_attention use the same array on streams that have no
// workspace of their own (gsdh_attention_workspace_create), so they allocate
// nothing either.
#include <mutex>

#include "gsd_internal.h"
#include "../../include/gsdhip.h"

using namespace gsd;

namespace {

// A 256-byte header (the device epoch word at byte 0, the error word at
// byte 8) and the split partial words of one launch (AttnArgs::ws).  Each
// GPU holds its own copy until the process ends, zero from the start; host
// code reaches it only through the address hipGetSymbolAddress returns on
// that device (NoAllocDev::ptr), never through the array's name.
constexpr size_t kScratchBytes = 8u << 20;
static __device__ __align__(256) unsigned long long scratch[kScratchBytes / 8];

// Per device: the scratch address (set once, with that device current).
// Nothing else is kept on the host: each launch takes its epoch from the
// header on the device, so graph replays of a captured call and calls of
// any shape never read one another's words.
struct NoAllocDev {
    unsigned long long* ptr = nullptr;
};
constexpr int kMaxDev = 64;
std::mutex g_mu;
NoAllocDev g_dev[kMaxDev];

// The scratch of the current device (its address on first use).
int scratch_ptr(hipStream_t stream, unsigned long long** out, const char* who) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail((int)e, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDev) return fail(-1, "%s: device %d beyond %d", who, dev, kMaxDev);
    std::lock_guard<std::mutex> lk(g_mu);
    NoAllocDev& d = g_dev[dev];
    if (!d.ptr) {
        // once per device, with that device current: the device address of
        // this GPU's copy of the array
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return fail((int)e, "%s: hipGetSymbolAddress: %s", who, hipGetErrorString(e));
        if (!p) return fail(-1, "%s: no device address for the scratch array", who);
        // the array starts at zero (static storage); outside graph capture
        // it is cleared once more by a fill kernel, stream-ordered before
        // the first launch that uses it
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(stream, &cs);
        if (e != hipSuccess) return fail((int)e, "%s: hipStreamIsCapturing: %s", who, hipGetErrorString(e));
        if (cs == hipStreamCaptureStatusNone) {
            e = launch_fill_u32(static_cast<unsigned*>(p), 0u, kScratchBytes / 4, stream);
            if (e != hipSuccess) return fail((int)e, "%s: clearing the scratch: %s", who, hipGetErrorString(e));
        }
        d.ptr = static_cast<unsigned long long*>(p);
    }
    *out = d.ptr;
    return 0;
}

}  // namespace

namespace gsd {

// A one-token attention launch on the current device's scratch: fills a.ws /
// a.dep / a.err (a.max_splits set) or fails for partials beyond it.
int attention_static_ws(hipStream_t stream, AttnArgs& a, int group, const char* who) {
    const size_t need = attention_ws_bytes(a.n_kv, a.max_splits, group, a.hd);
    if (need > kScratchBytes - kAttnWsHeader)
        return fail(-1,
                    "%s: %zu bytes of split partials (%d KV heads x %d splits x %d heads x %d dims) exceed the "
                    "%zu-byte static scratch; give the stream a workspace (gsdh_attention_workspace_create)",
                    who, need, a.n_kv, a.max_splits, group, a.hd, kScratchBytes - kAttnWsHeader);
    unsigned long long* p = nullptr;
    const int rc = scratch_ptr(stream, &p, who);
    if (rc) return rc;
    attention_use_ws(a, p);
    return 0;
}

// Reads and clears the error word of the current device's scratch (after the
// caller synchronised): 1 when a merge's bounded wait ran out since the last
// check.  Nothing to check before the scratch's first use.
int attention_static_error(int* was_set) {
    *was_set = 0;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail((int)e, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDev) return 0;
    unsigned long long* p = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        p = g_dev[dev].ptr;
    }
    if (!p) return 0;
    unsigned* ew = reinterpret_cast<unsigned*>(p + 1);
    unsigned v = 0;
    e = hipMemcpy(&v, ew, 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return fail((int)e, "reading the attention error word: %s", hipGetErrorString(e));
    if (v) {
        const unsigned zero = 0;
        e = hipMemcpy(ew, &zero, 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) return fail((int)e, "clearing the attention error word: %s", hipGetErrorString(e));
        *was_set = 1;
    }
    return 0;
}

}  // namespace gsd

extern "C" int gsdh_gqa_attention_noalloc(void* stream, const float* q, const uint16_t* k_cache,
                                          const uint16_t* v_cache, float* attn_out, int layer_idx, int pos,
                                          int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                                          float sm_scale) {
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return fail(-1, "attention_noalloc: head_dim %d not in {64,128,256}", head_dim);
    if (n_kv_heads <= 0 || n_heads % n_kv_heads || (8 % (n_heads / n_kv_heads)) != 0)
        return fail(-1, "attention_noalloc: n_heads %d / n_kv_heads %d is not a group size in {1,2,4,8}", n_heads,
                    n_kv_heads);
    if (pos < 0 || pos >= max_seq_len) return fail(-1, "attention_noalloc: pos %d outside 0..%d", pos, max_seq_len - 1);
    const int n = pos + 1, G = n_heads / n_kv_heads;
    AttnArgs a{};
    a.q = q; a.k_cache = k_cache; a.v_cache = v_cache; a.out = attn_out; a.pos_dev = nullptr; a.pos = pos;
    a.layer = layer_idx; a.n_heads = n_heads; a.n_kv = n_kv_heads; a.hd = head_dim; a.max_seq = max_seq_len;
    a.sm_scale = sm_scale;
    a.chunk = attention_chunk(n, n_kv_heads);
    a.max_splits = (n + a.chunk - 1) / a.chunk;
    attention_test_knobs(a);
    const int rc = attention_static_ws(static_cast<hipStream_t>(stream), a, G, "attention_noalloc");
    if (rc) return rc;
    const hipError_t e = launch_attention(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail((int)e, "attention_noalloc: %s", hipGetErrorString(e));
    return 0;
}
