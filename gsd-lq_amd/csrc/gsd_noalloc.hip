// gsd_noalloc.hip -- gsdh_gqa_attention_noalloc: the decode attention twin for
// callers that cannot allocate device memory (HIP graph capture, serving
// loops, harnesses that forbid hipMalloc).  The split partials that
// gsdh_gqa_attention keeps in a workspace it allocates live here in a
// file-scope device array instead.
#include <mutex>

#include "gsd_internal.h"
#include "../../include/gsdhip.h"

using namespace gsd;

namespace {

// The split partial words of one launch (AttnArgs::ws).  Each GPU holds its
// own copy until the process ends; host code reaches it only through the
// address hipGetSymbolAddress returns on that device (NoAllocDev::ptr),
// never through the array's name.
constexpr size_t kScratchBytes = 8u << 20;
static __device__ __align__(256) unsigned long long scratch[kScratchBytes / 8];

// Per device: the scratch address and the epoch of the last launch.  The
// array is cleared by a fill kernel before its first launch; every launch
// takes the next epoch, so words of earlier calls (of any shape) never match.
struct NoAllocDev {
    unsigned long long* ptr = nullptr;
    unsigned epoch = 0;
};
constexpr int kMaxDev = 64;
std::mutex g_mu;
NoAllocDev g_dev[kMaxDev];

}  // namespace

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
    const size_t need = attention_ws_bytes(n_kv_heads, a.max_splits, G, head_dim);
    if (need > kScratchBytes)
        return fail(-1,
                    "attention_noalloc: %zu bytes of split partials (%d KV heads x %d splits x %d heads x %d dims) "
                    "exceed the %zu-byte static scratch; use gsdh_gqa_attention",
                    need, n_kv_heads, a.max_splits, G, head_dim, kScratchBytes);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail((int)e, "attention_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDev) return fail(-1, "attention_noalloc: device %d beyond %d", dev, kMaxDev);
    std::lock_guard<std::mutex> lk(g_mu);
    NoAllocDev& d = g_dev[dev];
    if (!d.ptr) {
        // once per device, with that device current: the device address of
        // this GPU's copy of the array
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return fail((int)e, "attention_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
        if (!p) return fail(-1, "attention_noalloc: no device address for the scratch array");
        d.ptr = static_cast<unsigned long long*>(p);
        d.epoch = 0xFFFFFFF0u;   // cleared below before the first launch
    }
    if (d.epoch >= 0xFFFFFFF0u) {   // first call on the device, or the epoch about to wrap
        e = launch_fill_u32(reinterpret_cast<unsigned*>(d.ptr), 0u, kScratchBytes / 4, static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return fail((int)e, "attention_noalloc: clearing the scratch: %s", hipGetErrorString(e));
        d.epoch = 0;
    }
    a.ws = d.ptr;
    a.counters = nullptr;
    a.epoch = ++d.epoch;
    e = launch_attention(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail((int)e, "attention_noalloc: %s", hipGetErrorString(e));
    return 0;
}
