/*
 * gsdhip.h -- C ABI of libgsdhip.so, the MI355X (gfx950) GSD-LQ decode engine.
 *
 * Two layers:
 *
 *  1. Operator twins of the reference CPU engine (gsd_lq_v2/gsd_lq_cpu_engine.c).
 *     Same names with a gsdh_ prefix, same argument order and meaning, plus a
 *     leading stream argument; every pointer is a DEVICE pointer in the
 *     reference's own data layout; the call is asynchronous on `stream`
 *     (a hipStream_t, 0 = null stream) and returns 0 or a nonzero status
 *     whose text gsdh_last_error() returns.  They replace the ctypes bindings
 *     of gsd_lq_v2/gsd_lq_cpu_runtime.py:91-108 and the OpenCL kernels of
 *     gsd_lq_v2/run_gpu_native_chat.py:101-421 one for one.
 *
 *  2. A model context that owns the packed weights in the engine's device
 *     layout, the fp16 KV cache and the activations, and runs a whole token
 *     (32 layers, ~195 kernels captured in one HIP graph) per call.  It replaces
 *     GPUMistralV2Model.forward_token (run_gpu_native_chat.py:892-969) and the
 *     per-kernel Python launches of _matvec_gpu (run_gpu_native_chat.py:858-890).
 *
 * No torch types cross this boundary: plain pointers, sizes and ints.
 */
#ifndef GSDHIP_H
#define GSDHIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Library status                                                            */
/* ------------------------------------------------------------------------ */

/* Text of the last error raised on the calling thread ("" if none). */
const char* gsdh_last_error(void);

/* Name and total memory of the current HIP device (the reference exposes the
 * OpenCL device name and VRAM, run_gpu_native_chat.py:503-509). */
int gsdh_device_info(char* name, int name_len, uint64_t* total_bytes, int* n_cu);

/* Device memory helpers for callers without another allocator. */
int gsdh_malloc(void** ptr, uint64_t nbytes);
int gsdh_free(void* ptr);
int gsdh_memcpy_h2d(void* dst, const void* src, uint64_t nbytes, void* stream);
int gsdh_memcpy_d2h(void* dst, const void* src, uint64_t nbytes, void* stream);
/* Waits for the stream; then returns -2 (text in gsdh_last_error) when a
 * stand-alone attention launch on this device (the gsdh_*attention* twins
 * below) gave up a bounded wait for a split's partials since the last check,
 * whose output is then undefined: like a kernel fault, the asynchronous
 * failure surfaces at the next synchronisation (the reference raises
 * RuntimeError on launch errors, run_gpu_native_chat.py:648-649). */
int gsdh_stream_sync(void* stream);
/* Streams and graph capture for callers without another HIP binding (no
 * reference counterpart; the reference's single OpenCL queue is
 * run_gpu_native_chat.py:521).  Streams are non-blocking and of the default
 * priority; gsdh_stream_destroy also frees the stream's attention workspace. */
int gsdh_stream_create(void** stream_out);
int gsdh_stream_destroy(void* stream);
int gsdh_stream_begin_capture(void* stream);
int gsdh_stream_end_capture(void* stream, void** graph_exec_out);
int gsdh_graph_replay(void* graph_exec, void* stream);
/* Plain device-to-device copy by a 16-byte streaming kernel (nbytes % 16 == 0);
 * used to calibrate HBM traffic counters against a known byte count. */
int gsdh_stream_copy(void* stream, void* dst, const void* src, uint64_t nbytes);

/* ------------------------------------------------------------------------ */
/* 1. Operator twins of gsd_lq_cpu_engine.c                                  */
/* ------------------------------------------------------------------------ */

/* gsd_cpu_rmsnorm (gsd_lq_cpu_engine.c:66-82): out = x * (1/sqrtf(mean(x^2)+eps)) * w */
int gsdh_rmsnorm(void* stream, const float* x, const float* weight, float* out, int dim, float eps);

/* gsd_cpu_vec_add (gsd_lq_cpu_engine.c:84-94): y = a + b */
int gsdh_vec_add(void* stream, float* y, const float* a, const float* b, int dim);

/* gsd_cpu_swiglu (gsd_lq_cpu_engine.c:96-108): out = gate/(1+exp(-gate)) * up */
int gsdh_swiglu(void* stream, const float* gate, const float* up, float* out, int dim);

/* gsd_cpu_lowrank_proj (gsd_lq_cpu_engine.c:110-127):
 * tmp_k[j] = S[j] * sum_c x[c] * fp16(Vt[j,c]), j < k_dim <= 16 */
int gsdh_lowrank_proj(void* stream, const float* x, const uint16_t* Vt, const float* S,
                      float* tmp_k, int k_dim, int cols);

/* gsd_cpu_hex2d_matvec (gsd_lq_cpu_engine.c:129-183):
 * y[r] = sum_p (T[code].x*x[2p] + T[code].y*x[2p+1]) * fp16(scale[r*cols/64 + p/32])
 *      + sum_{kinks of r} delta * x[col] + sum_j fp16(U[r,j]) * tmp_k[j]
 * codes: u8 [rows*cols/2]; scales: fp16 bits [rows*cols/64]; xy_table: float2
 * [n_pts]; cols must be a positive multiple of 64 and n_pts <= 256. */
int gsdh_hex2d_matvec(void* stream, const float* x, const uint8_t* codes, const uint16_t* scales,
                      const float* xy_table, const uint16_t* U, const float* tmp_k,
                      const uint32_t* kink_row_ptr, const uint16_t* kink_cols,
                      const float* kink_deltas, float* y, int rows, int cols, int k_dim, int n_pts);

/* gsd_cpu_rope_and_store_kv (gsd_lq_cpu_engine.c:185-262): rotates q in place
 * and k, stores fp16(k') and fp16(v) at cache[((layer*max_seq+pos)*n_kv+h)*hd+d].
 * cos/sin are evaluated on the host with the C library exactly as the
 * reference does, so the cache bits match it for equal inputs. */
int gsdh_rope_and_store_kv(void* stream, float* q, const float* k, const float* v,
                           uint16_t* k_cache, uint16_t* v_cache, int layer_idx, int pos,
                           int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                           float rope_theta, int interleaved);

/* gsd_cpu_gqa_attention (gsd_lq_cpu_engine.c:264-330): softmax(q.K/scale)V
 * over cached positions 0..pos, split over the context (flash-decoding);
 * head_dim must be 64, 128 or 256; n_heads/n_kv_heads must be 1, 2, 4 or 8.
 * Allocates nothing: the split partials go to the stream's workspace when
 * gsdh_attention_workspace_create made one, else to the library's static
 * per-GPU scratch (the limit of gsdh_gqa_attention_noalloc below; calls on
 * that scratch that overlap on one GPU race).  Each launch takes its epoch
 * on the device, so a captured call replays correctly. */
int gsdh_gqa_attention(void* stream, const float* q, const uint16_t* k_cache,
                       const uint16_t* v_cache, float* attn_out, int layer_idx, int pos,
                       int n_heads, int n_kv_heads, int head_dim, int max_seq_len, float sm_scale);

/* A workspace of its own for the attention twins on `stream` (calls on
 * different streams may then overlap), sized for contexts up to max_seq_len
 * positions of this head shape; allocated here, once, and freed by
 * gsdh_attention_workspace_destroy (or gsdh_stream_destroy).  The caller
 * owns its lifetime, as it owns every buffer of the reference's engine
 * (gsd_lq_cpu_runtime.py:91-108).  No reference counterpart.
 * gsdh_attention_workspace_bytes: its size (0 for an invalid shape). */
uint64_t gsdh_attention_workspace_bytes(int n_kv_heads, int n_heads, int head_dim, int max_seq_len);
int gsdh_attention_workspace_create(void* stream, int n_kv_heads, int n_heads, int head_dim,
                                    int max_seq_len);
int gsdh_attention_workspace_destroy(void* stream);

/* gsd_cpu_rope_and_store_kv followed by gsd_cpu_gqa_attention
 * (gsd_lq_cpu_engine.c:185-330), the two calls of one decode step's
 * attention (gsd_lq_cpu_runtime.py:325-361), in one launch: q is rotated in
 * place, fp16(k') and fp16(v) are stored at position pos, and attn_out is the
 * attention over positions 0..pos.  Same results, bit for bit, as
 * gsdh_rope_and_store_kv then gsdh_gqa_attention on the same stream (the
 * rotation uses the same host cos/sin and no contraction).  One launch for
 * head_dim 64 or 128, 1, 2 or 4 query heads per KV head and up to 8192
 * positions; other shapes run the two launches. */
int gsdh_rope_store_gqa_attention(void* stream, float* q, const float* k, const float* v,
                                  uint16_t* k_cache, uint16_t* v_cache, float* attn_out,
                                  int layer_idx, int pos, int n_heads, int n_kv_heads, int head_dim,
                                  int max_seq_len, float rope_theta, int interleaved, float sm_scale);

/* gsd_cpu_gqa_attention (gsd_lq_cpu_engine.c:264-330) for n_tokens
 * consecutive prompt tokens at once, on the matrix cores: token t (query rows
 * q[t][n_heads][head_dim], RoPE applied, its K/V rows already stored at
 * position pos0 + t) attends over cache positions 0 .. pos0 + t, and
 * attn_out[t][n_heads][head_dim] is what gsdh_gqa_attention at pos0 + t
 * returns (to fp32 rounding).  The reference prefills token by token
 * (run_gpu_native_chat.py:1128-1130); this is the batched form the model's
 * prefill uses.  head_dim 64, 128 or 256; n_heads/n_kv_heads 1, 2, 4 or 8;
 * pos0 + n_tokens <= max_seq_len.  No workspace, nothing allocated. */
int gsdh_prefill_attention(void* stream, const float* q, const uint16_t* k_cache,
                           const uint16_t* v_cache, float* attn_out, int layer_idx, int pos0,
                           int n_tokens, int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                           float sm_scale);

/* gsd_cpu_gqa_attention for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Same arguments and results as
 * gsdh_gqa_attention, but the split partials always live in a static 8 MiB
 * device array of the library (one per GPU, kept until the process ends),
 * so the call allocates nothing; each launch takes its epoch from a word in
 * that array on the device, so graph replays of a captured call are
 * correct.  Limit: n_kv_heads * splits * (n_heads/n_kv_heads) * (head_dim +
 * 2) * 8 bytes <= 8 MiB - 256, where n = pos + 1 positions split as: one
 * split up to 128 positions; beyond, chunks of the smallest of 64, 128, 256
 * that is >= ceil(n * n_kv_heads / 256) (256 at most), splits = ceil(n /
 * chunk).  E.g. 8 KV heads x 4 x 128 dims at context 8192 (32 splits of
 * 256) use 1.1 MB.  Larger calls fail with an error.  All calls on one GPU
 * share the array (with gsdh_gqa_attention on streams without a workspace):
 * calls that overlap on one GPU (different streams, or threads) race.  A
 * merge that gave up waiting is reported by gsdh_stream_sync. */
int gsdh_gqa_attention_noalloc(void* stream, const float* q, const uint16_t* k_cache,
                               const uint16_t* v_cache, float* attn_out, int layer_idx, int pos,
                               int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                               float sm_scale);

/* Bit-exact unpack of codes: idx[i] = codes[i], r01[2i..2i+1] = integer
 * lattice fields (r0, r1) of codeword idx[i] in the radius-R enumeration.
 * Used to check the device decode path (no reference counterpart; the
 * enumeration is gsd_lq_cpu_runtime.py:111-118). */
int gsdh_unpack_codes(void* stream, const uint8_t* codes, int64_t n, int radius,
                      int32_t* idx_out, int8_t* r01_out);

/* Greedy branch of sample_token (gsd_lq_cpu_runtime.py:422-425):
 * nan_to_num(nan=-1e4, posinf=100, neginf=-1e4), then the first index of the
 * maximum.  logits: device f32 [n]; writes the token to device *token_out and
 * the top1 - top2 margin of the cleaned values to device *margin_out.  One
 * block: calls on any streams may overlap. */
int gsdh_greedy_argmax(void* stream, const float* logits, int n, int* token_out, float* margin_out);
/* The same greedy step over 32 blocks, the form that ends every greedy step
 * of the model context (one block's loads of a 32768-entry vocabulary are
 * bound by one CU's outstanding misses).  words: device u64 [96], counters:
 * device u32 [32], both zero before their first call; calls that share them
 * must not overlap (one stream).  Same outputs as gsdh_greedy_argmax
 * (gsd_lq_cpu_runtime.py:422-425). */
int gsdh_greedy_argmax_split(void* stream, const float* logits, int n, int* token_out, float* margin_out,
                             uint64_t* words, uint32_t* counters);

/* ------------------------------------------------------------------------ */
/* 2. Model context (replaces GPUMistralV2Model's device side)              */
/* ------------------------------------------------------------------------ */

typedef struct gsdh_model gsdh_model;

typedef struct gsdh_model_config {
    int n_layers, hidden, ffn, n_heads, n_kv_heads, head_dim, vocab;
    int max_seq_len;          /* KV capacity (reference: 2048) */
    int rope_interleaved;     /* 1 = (2i, 2i+1) pairs, 0 = (i, i+hd/2) */
    float rms_eps, rope_theta;
} gsdh_model_config;

/* Tensor slots of a layer, in the order of run_gpu_native_chat.py:822-828. */
enum { GSDH_Q = 0, GSDH_K, GSDH_V, GSDH_O, GSDH_GATE, GSDH_UP, GSDH_DOWN, GSDH_LM_HEAD };

int gsdh_model_create(const gsdh_model_config* cfg, gsdh_model** out);
int gsdh_model_destroy(gsdh_model* m);

/* Dense tensors from host memory.  embed: fp16 bits [vocab, hidden];
 * norms: f32 [hidden]; layer = -1 for output_norm.  These and
 * gsdh_model_set_hex fail once the model is finalized. */
int gsdh_model_set_embedding(gsdh_model* m, const uint16_t* embed_f16);
int gsdh_model_set_norm(gsdh_model* m, int layer, int which /*0 attn, 1 ffn*/, const float* w);

/* A packed tensor from host memory in .gsd2 layout (fields as in the file).
 * layer is ignored for GSDH_LM_HEAD.  Validates shapes and that every code is
 * < n_pts; transcodes into the engine's device layout. */
int gsdh_model_set_hex(gsdh_model* m, int layer, int slot, int radius, int rows, int cols,
                       int k_dim, const uint8_t* codes, const uint16_t* scales,
                       const uint32_t* row_ptr, const uint16_t* kink_cols,
                       const float* kink_deltas, int64_t nk, const uint16_t* U, const float* S,
                       const uint16_t* Vt);

/* After every tensor is set: checks completeness, builds the RoPE tables and
 * the per-token HIP graphs that forward_token / generate_greedy replay: one
 * launch per fused phase (q/k/v + RoPE + KV append with the decode attention
 * of short contexts, attention, o, gate/up + SwiGLU, down, head, argmax), in
 * place of the reference's per-token sequence of OpenCL launches
 * (run_gpu_native_chat.py:892-969). */
int gsdh_model_finalize(gsdh_model* m);

/* Device bytes held by the model (weights + KV cache + activations). */
uint64_t gsdh_model_device_bytes(gsdh_model* m);

/* One token through every layer at position pos; when want_logits, copies the
 * vocab-sized f32 logits into logits_host (may be NULL to skip the copy) and
 * returns the greedy token (first argmax) in *argmax_out (may be NULL). */
int gsdh_forward_token(gsdh_model* m, int token_id, int pos, int want_logits,
                       float* logits_host, int* argmax_out);

/* Prefill prompt[0..n_prompt) at positions start_pos.., then n_new greedy
 * steps entirely on the device; writes the generated ids and the top1-top2
 * logit margin of every step.  The prompt goes through gsdh_model_prefill's
 * batched forward (gsdh_model_set_prefill(m, 0): token by token through the
 * decode graph, as the reference does). */
int gsdh_generate_greedy(gsdh_model* m, const int* prompt, int n_prompt, int start_pos, int n_new,
                         int* tokens_out, float* margins_out);

/* Batched prefill (the reference prefills token by token,
 * run_gpu_native_chat.py:1128-1130, reusing a cached prefix, :1112-1115):
 * tokens[0..n) at positions start_pos.. through every layer at once, in
 * chunks of 128 tokens: per layer the q/k/v, o, gate/up and down projections
 * of all the chunk's tokens on the matrix cores (activations as fp16 high +
 * low parts, fp32 accumulation, RMSNorm / rank-k / kink terms as the
 * reference computes them), RoPE and fp16 K/V append at every position, and
 * causal attention of each token over the cache positions 0..its own (a
 * cached prefix below start_pos is reused).  When want_logits, the last
 * token's logits are copied to logits_host (may be NULL) and its greedy
 * token to *argmax_out; the step state then holds position start_pos + n
 * for the next decode step.  Allocates nothing (the workspace is the
 * model's, sized at finalize).  Synchronous. */
int gsdh_model_prefill(gsdh_model* m, const int* tokens, int n, int start_pos, int want_logits,
                       float* logits_host, int* argmax_out);
/* 1: generate_greedy prefills with gsdh_model_prefill (the default); 0: one
 * decode-graph launch per prompt token. */
int gsdh_model_set_prefill(gsdh_model* m, int batched);

/* Batched projection for prefill on the matrix cores: Y[m][r] = (W x_m)[r] for
 * the packed tensor (layer, slot) of the model and M tokens at once, kinks and
 * rank-k terms included (each token's rank-k projection from its bf16 row).
 * X: device bf16 [M][cols]; Y: device fp32 [M][rows]; asynchronous on the
 * model stream (gsdh_stream_sync(gsdh_model_stream(m)) to wait).  The
 * arithmetic is the fused matvec's (run_gpu_native_chat.py:196-267 /
 * gsd_lq_cpu_engine.c:129-183) per token, with the token's (u, v) pair terms
 * rounded once to fp16 (about 1e-4 relative).  No counterpart in the
 * reference, which prefills token by token (run_gpu_native_chat.py:1128-1130).
 * M <= 512 per call; the staging lives in the model's workspace (sized at
 * finalize), so the call allocates nothing and can be graph-captured. */
int gsdh_model_matmul(gsdh_model* m, int layer, int slot, const uint16_t* X, int M, float* Y);
/* The same for n <= 3 tensors of `layer` that read the same X (q, k, v or
 * gate, up): X's operands are prepared once, then each tensor's projection
 * runs into Y[i] (device fp32 [M][rows_i]).  Equal to n gsdh_model_matmul
 * calls, bit for bit. */
int gsdh_model_matmul_shared(gsdh_model* m, int layer, const int* slots, int n, const uint16_t* X, int M,
                             float* const* Y);
/* The tiling gsdh_model_matmul and the batched prefill use for M tokens of a
 * rows x cols tensor on the current device: token groups of 16 per block
 * (*tg: 1, 2, 4, 8), row blocks of 16 per wave (*rbw) and column splits
 * (*nsplit).  A diagnostic (tests name the tiles they run); no reference
 * counterpart. */
int gsdh_matmul_plan(int M, int rows, int cols, int* tg, int* rbw, int* nsplit);

/* The codes of packed tensor (layer, slot) as the device holds them, decoded
 * back to the file's u8 [rows][cols/2] order on the device by the same tile
 * decoding the matvec kernels use (one byte per code for radius 7-8, seven
 * bits for radius <= 6) and copied to host `codes_out` (rows*cols/2 bytes);
 * synchronous.  A check that decoding is bit-exact (the reference reads the
 * u8 codes directly, run_gpu_native_chat.py:806, gsd_lq_cpu_runtime.py:191;
 * no counterpart entry point). */
int gsdh_model_read_codes(gsdh_model* m, int layer, int slot, uint8_t* codes_out);

/* Runs the model's fused matvec launches of `layer` on the model stream with
 * the current activations, without attention or synchronisation.  Mask bit i
 * = projection set i of {qkv, o, gate+up, down} (4 | 8 together run as one
 * launch, and 2 | 4 | 8 too, where gsdh_model_fused_ffn says so):
 *   1: q, k, v of rmsnorm(x) * attn_norm, RoPE(q) -> q, fp16 RoPE(k) and v
 *      appended to the cache at the step position (run_gpu_native_chat.py:
 *      899-925);  2: x += W_o attn;  4: h = silu(W_gate x') * (W_up x') with
 *      x' = rmsnorm(x) * ffn_norm;  8: x += W_down h (chat.py:927-956).
 * mask 16 alone runs the head instead: logits = W_lm rmsnorm(x) * out_norm
 * (chat.py:962-968), layer ignored.  Used by the benchmark and by the
 * full-shape parity tests of each launch. */
int gsdh_model_run_linear(gsdh_model* m, int layer, int mask);

/* How `layer`'s o, gate/up and down projections run (no counterpart entry
 * point): 2 = o, gate/up and down in one launch (mask 2 | 4 | 8 of
 * gsdh_model_run_linear and every decode token: each block forms 16 rows of
 * x + W_o attn and hands them over as tagged words, then h of its 64 FFN
 * rows, then that block's 64 columns of W_down as partial sums that the
 * launch reduces in block order; gsd_lq_cpu_runtime.py:376-404); 1 = gate/up
 * and down in one launch, o in its own (GSD_FUSED_OFFN=0, o not square or
 * of another radius or rank; also mask 4 | 8 without 2); 0 = three launches
 * (GSD_FUSED_FFN=0, shapes beyond the launch's grid, tensors of different
 * radii or of ranks other than all 0 / all 2); negative on a bad argument. */
int gsdh_model_fused_ffn(gsdh_model* m, int layer);

/* Activation vectors of the model context (f32): x [hidden], q [n_heads*hd],
 * k / v [n_kv*hd], attn [n_heads*hd], h [ffn], logits [vocab].  write = 1
 * copies host -> device, 0 device -> host; nbytes must be the vector's size.
 * Synchronous (waits for the model stream first).  With gsdh_model_set_step
 * and gsdh_model_read_kv they let a harness feed one launch of
 * gsdh_model_run_linear and read its result, as the reference's ctypes
 * harness feeds NumPy buffers to each gsd_cpu_* call
 * (gsd_lq_cpu_runtime.py:316-404).  No counterpart in the reference. */
enum { GSDH_VEC_X = 0, GSDH_VEC_Q, GSDH_VEC_K, GSDH_VEC_V, GSDH_VEC_ATTN, GSDH_VEC_H, GSDH_VEC_LOGITS };
int gsdh_model_vector(gsdh_model* m, int which, int write, void* host, uint64_t nbytes);
/* Step state read by the launches: token id and position (RoPE angle and
 * KV slot of the qkv launch).  Synchronous. */
int gsdh_model_set_step(gsdh_model* m, int token_id, int pos);
/* The fp16 K and V cache rows [n_kv*hd] of (layer, pos) to host memory. */
int gsdh_model_read_kv(gsdh_model* m, int layer, int pos, uint16_t* k_out, uint16_t* v_out);

/* Graph capture of an arbitrary sequence of the model's own launches on its
 * stream, for timing: begin, issue calls, end -> replay n times. */
int gsdh_model_capture_begin(gsdh_model* m);
int gsdh_model_capture_end(gsdh_model* m, void** graph_exec_out);
int gsdh_graph_launch(gsdh_model* m, void* graph_exec, int n_times);
int gsdh_graph_destroy(void* graph_exec);
/* n_times launches of graph_exec on the model stream bracketed by HIP events;
 * *ms_out = elapsed milliseconds between the two events. */
int gsdh_graph_time(gsdh_model* m, void* graph_exec, int n_times, float* ms_out);
void* gsdh_model_stream(gsdh_model* m);

#ifdef __cplusplus
}
#endif
#endif /* GSDHIP_H */
