// gsd_internal.h -- launch interface between the kernels (gsd_kernels.hip) and
// the C ABI / model runtime (gsd_capi.hip).  Internal to libgsdhip.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gsd {

constexpr int kMaxSeg = 3;        // q, k, v share one launch
constexpr int kMaxRank = 16;      // tmp_k scratch of the reference is 16 floats
constexpr int kTableSlots = 256;  // LDS codebook slots (codes are u8)

// One packed tensor of a fused matvec launch.  All pointers are device
// pointers in the .gsd2 field layout (codes row-major u8 pairs, fp16 scales
// per 64 weights, CSR kinks, U [rows,k], Vt [k,cols]).
struct HexSeg {
    const uint8_t* codes;
    const uint16_t* scales;
    const uint32_t* row_ptr;   // null: no kinks
    const uint16_t* kcols;
    const float* kdel;
    const uint16_t* U;         // k > 0
    const uint16_t* Vt;        // k > 0 and tmp_k == null: computed in-kernel
    const float* S;
    const float* tmp_k;        // k > 0: precomputed low-rank projection, or null
    const float* table;        // float2 [n_pts]: codeword points (generic path)
    // half2 [n_pts] integer fields (r0, r1) of the A2 codewords, whose points
    // are (r0 + r1/2, r1*sqrt(3)/2); non-null in every segment selects the
    // lattice path (requires scale_t = 1)
    const uint32_t* fields;
    // tiled device layout of the MFMA path (hexmv4):
    //   codes_t  [ceil(rows/16)][ceil(cols/128)][64 lanes][16 B]
    //   scales_t [ceil(rows/16)][ceil(cols/128)][16 rows] fp16 pairs
    // lane l holds row 16*rb + (l & 15); its byte j is pair 64c + 8(l >> 4) + j
    // (j < 8) or 64c + 32 + 8(l >> 4) + j - 8 (j >= 8) of that row; the scale
    // pair holds the two 64-weight blocks of the chunk.  Padding is code 0 /
    // scale 0.
    const uint4* codes_t;
    const uint32_t* scales_t;
    float* out;
    int rows, k, n_pts, batch0;
};

enum HexEpilogue : int {
    kEpiStore = 0,     // out[r] = y[r]
    kEpiResidual = 1,  // out[r] = resid[r] + y[r]          (x += W x')
    kEpiSwiGLU = 2,    // seg0/seg1 paired rows: out[r] = silu(y0[r]) * y1[r]
    kEpiRopeKV = 3,    // q/k/v segments: RoPE(q), RoPE(k) -> fp16 cache, v -> fp16 cache
};

// RoPE + KV append state for kEpiRopeKV (and the stand-alone rope kernel).
struct RopeKV {
    const float2* cs;       // [max_seq][hd/2] (cos, sin); row pos used
    const int* pos_dev;     // device position (graph replay); null -> pos
    int pos;
    uint16_t* k_cache;
    uint16_t* v_cache;
    int layer, n_heads, n_kv, hd, max_seq, interleaved;
};

struct HexArgs {
    HexSeg seg[kMaxSeg];
    int nseg;
    const float* x;        // input vector [cols]
    const float* norm_w;   // non-null: input = rmsnorm(x) * norm_w
    float eps;
    float* resid;          // kEpiResidual target (read-modify-write)
    int cols;
    int nbatch;            // row batches in total
    int epilogue;
    int scale_t;           // scales layout: 0 = row-major [rows][cols/64] (file),
                           // 1 = [ceil(rows/4)][cols/64][4] (4 rows per 8-byte load)
    RopeKV rope;           // kEpiRopeKV: interleaved RoPE of q/k rows, fp16 K/V append
    // In-launch rank-k projection (segments with k > 0 and tmp_k == null):
    // block b < sum(k) computes one tmp_k value and publishes it as one 64-bit
    // word pub[b] = 1 << 32 | float bits (a single atomic store, so a reader
    // sees 0 or the whole value, and no fence is needed).  Every block with
    // rows to do polls the words before its first epilogue.  The words must
    // be zero when the launch starts (each launch of a sequence has its own).
    unsigned long long* pub;
    unsigned* err;             // set to 1 when the wait exceeds its bound
    // Decode attention in the q/k/v launch (kEpiRopeKV, positions < 256):
    // the last nkv blocks of the grid are attention blocks, one per KV head.
    // The q/k/v epilogue publishes its outputs as 64-bit words, tag << 32 |
    // bits (q rows as fp32; the new K and V rows, as written to the cache, as
    // fp16 pairs), one relaxed device-scope store each; the attention block
    // of a KV head waits for the words of its rows to carry the launch's tag
    // = *epoch_dev * 64 + layer + 1 (epoch_dev: the token counter the
    // embedding launch advances; layers < 64), so nothing is ever cleared.
    struct FusedAttn {
        unsigned long long* words;   // [n_heads * hd + n_kv * hd]: q rows, K pairs, V pairs
        float* out;                  // attention output [n_heads * hd]
        const unsigned* epoch_dev;
        float sm_scale;
        int nkv;                     // 0: no attention blocks
        int span;                    // positions the blocks cover: 64, 128 or 256 (0: 256)
    } fa;
    // hexmv4 launch plan, filled in by launch_hexmv4 (callers leave it zero):
    // per-launch constants the kernel would otherwise derive with integer
    // divisions ahead of its first loads
    struct Mv4Plan {
        int P;                 // 128-column chunks per wave and unit
        int wr_log2;           // log2 of the waves of a row-block group
        int nunits;            // row-block units of the launch
        int ub1, ub2;          // first units of segments 1 and 2
        int units_q, units_r;  // units of matvec block b: units_q + (b < units_r)
        int nw;                // matvec waves per block (blocks may be larger: fa)
        // paired gate/up launches: blocks b < su take, after their units_q
        // whole units, half of unit su_u0 + b / 2 (rows 8 (b & 1) .. + 7 of
        // gate and up; all waves of the block over the columns), so that
        // every block streams the same bytes (0: no half units)
        int su, su_u0;
    } mv;
};

constexpr int kLeadMax = kMaxSeg * kMaxRank;   // publishing blocks per launch

// The feed-forward block of one decode token in one launch
// (gsd_lq_cpu_runtime.py:380-404: x += W_down (silu(W_gate x') * (W_up x')),
// x' = rmsnorm(x) * ffn_norm).  Block b < nb owns FFN rows 64 b .. 64 b + 63:
// it forms those rows of gate and up (four 16-row units of each), their
// SwiGLU values h, then the down product of its own h over every output row,
// W_down[:, 64 b .. 64 b + 63] h[64 b ..], as partial sums (split-K): no
// block waits for another's h.  The partials go out as 64-bit words tag << 32
// | float bits (relaxed device-scope stores); block s < nslices then sums
// rows 16 s .. 16 s + 15 over every block's words in block order
// (deterministic), adds the rank-k and kink terms and the residual, and
// writes x.  Every block of the grid is resident at once (grid <= CU count,
// one block per CU), so the wait for the words ends (bounded: a timeout sets
// *err).  The tag is the launch count + 1: block b reads its own counter
// ctr[b] and stores it plus one (no other block reads ctr[b], and every block
// of every launch advances its own once, so all counters agree), so words of
// other launches never match and nothing is cleared (the counters wrap after
// 2^32 launches of one model).  Zero ctr and words at allocation.
struct FfnArgs {
    // gate / up in the tiled matvec layout (HexSeg::codes_t / scales_t)
    const unsigned char* gcodes;
    const uint32_t* gscales;
    const unsigned char* ucodes;
    const uint32_t* uscales;
    // down as column slabs: slab b = columns 64 b .. 64 b + 63, its step sd =
    // rows 32 sd .. 32 sd + 31 as one tile of 64 lanes x 16 codes; lane l
    // holds row 32 sd + (l & 15) (codes j < 8) and row 32 sd + 16 + (l & 15)
    // (j >= 8), pair 8 (l >> 4) + (j & 7) of the slab; the scale word holds
    // the fp16 scales of those two rows' 64-weight block
    const unsigned char* dcodes;
    const uint32_t* dscales;
    const uint32_t* fields;   // (r0, r1) fp16 pairs, padded to 256 entries
    int n_pts;
    // CSR kinks (row_ptr null: none) and rank-2 factors (R2 kernels)
    const uint32_t* g_rp;
    const uint16_t* g_kc;
    const float* g_kd;
    const uint32_t* u_rp;
    const uint16_t* u_kc;
    const float* u_kd;
    const uint32_t* d_rp;
    const uint16_t* d_kc;
    const float* d_kd;
    const uint16_t* gU;
    const uint16_t* uU;
    const uint16_t* dU;
    const float* gS;
    const float* uS;
    const float* dS;
    const uint16_t* gVt;
    const uint16_t* uVt;
    const uint16_t* dVt;
    // OF (ocodes non-null): the o projection first, x += W_o attn (o in
    // the tiled layout, qd == hidden columns), its rows formed by block
    // s < nslices 16 at a time and handed to every block as tagged words
    const unsigned char* ocodes;
    const uint32_t* oscales;
    const uint32_t* o_rp;
    const uint16_t* o_kc;
    const float* o_kd;
    const uint16_t* oU;
    const float* oS;
    const uint16_t* oVt;
    const float* attn;
    int qd;
    float* x;                    // residual stream: read, then x += W_down h
    const float* norm_w;         // ffn_norm
    float eps;
    float* h;                    // the SwiGLU values (written for inspection)
    unsigned long long* words;   // [nb][hpad] partials, [nb][2] rank words, [ffn] h words, [hidden] x words
    unsigned* ctr;               // [grid] launch counters, one per block
    unsigned* err;
    int hidden, ffn;
    int nb;          // working blocks: ffn / 64
    int nslices;     // reducing blocks: hidden / 16
    int hpad;        // row stride of the partial words (nslices * 16)
    int nc;          // 128-column chunks of x (hidden / 128)
    int nrb;         // 16-row blocks of gate / up
    int ns2;         // 32-row steps of a down slab
    int spin_limit;  // polling rounds before a wait counts as timed out
};
hipError_t launch_ffn(const FfnArgs& a, hipStream_t stream);
// words an FfnArgs::words buffer needs for a model shape, and the counters
size_t ffn_words(int hidden, int ffn);
constexpr int kFfnMaxGrid = 1024;
// whether launch_ffn covers the shape (grid within the CU count, chunking)
bool ffn_supported(int hidden, int ffn);

// Launches (all asynchronous on `stream`).
hipError_t launch_hexmv(const HexArgs& a, hipStream_t stream);
// MFMA matvec over the tiled layout (codes_t / scales_t / fields of every
// segment); same epilogues, norm and rank-k handling as launch_hexmv.
hipError_t launch_hexmv4(const HexArgs& a, hipStream_t stream);

// Batched projection (prefill) on the matrix cores: Y[m][r] = W x_m for M
// tokens, W one packed tensor in the tiled layout.  X is bf16 [M][cols];
// xa is the fp16 A-operand staging of X (hexmm_xa_bytes), xs the per-token
// descale factors [ceil(M/16)*16]; tmp_k [M][k] the tokens' rank-k values
// (null when k == 0).
struct MatmulArgs {
    HexSeg w;                  // codes_t, scales_t, fields, rows, n_pts, kinks, U, k
    const uint16_t* X;         // bf16 input (hl == 0; the kink terms read it)
    uint4* xa;
    float* xs;
    const float* tmp_k;
    float* Y;
    float* part;               // split-K partials [nsplit][ceil(M/16)*16][rows] (nsplit > 1)
    int M, cols;
    int nsplit;                // column splits (1: blocks write Y directly)
    int tg, rbw;               // tiling (hexmm_plan)
    // hl = 1: xa holds each token's (u, v) as fp16 high + low parts (about
    // 2^-22 relative, as the batch-1 matvec) prepared by launch_batch_prep,
    // two MFMAs per step; the kink terms read Xf (fp32 [M][cols], the
    // prepared input).  accumulate = 1: Y[m][row] += y (residual add).
    int hl;
    const float* Xf;
    int accumulate;
    // hl == 0: xa / xs already hold X's operands (an earlier launch_hexmm of
    // the same X, or launch_hexmm_xprep): the operand prep is skipped
    int prepped;
};
// The single-rounding fp16 operands of bf16 X [M][cols] into xa / xs (the
// prep launch_hexmm runs first), for several tensors that read the same X.
hipError_t launch_hexmm_xprep(const uint16_t* X, int M, int cols, uint4* xa, float* xs, hipStream_t stream);
size_t hexmm_xa_bytes(int M, int cols, int hl = 0);
// Operands of M tokens for the batched projections that share one input
// (q/k/v, gate/up, o, down): x' = rmsnorm(x) * norm_w (as
// gsd_lq_cpu_engine.c:66-82; norm_w null: x' = x) into xn (fp32 [M][cols]),
// the hi/lo fp16 MFMA fragments of (u, v) = (x'a, x'a / 2 + x'b sqrt(3) / 2)
// after a per-token power-of-two prescale (xa, descale xs), and the rank-k
// projections tmp[g][m * k[g] + j] = S_g[j] * sum_c x'[c] Vt_g[j][c] of up to
// kMaxSeg tensors (gsd_lq_cpu_engine.c:110-127).
struct BatchPrep {
    const float* X;
    int ldx;                   // row stride of X (floats)
    const float* norm_w;
    float eps;
    int M, cols;
    uint4* xa;
    float* xs;
    float* xn;
    const uint16_t* Vt[kMaxSeg];
    const float* S[kMaxSeg];
    int k[kMaxSeg];
    float* tmp[kMaxSeg];
};
hipError_t launch_batch_prep(const BatchPrep& p, hipStream_t stream);
// hexmm over operands launch_batch_prep made (a.hl = 1): no operand prep here
hipError_t launch_hexmm_prepared(const MatmulArgs& a, hipStream_t stream);
// X[m][:] = fp16 embedding row of tokens[m] (fp32 [M][hidden])
hipError_t launch_embed_rows(const uint16_t* embed, const int* tokens, int M, float* X, int hidden,
                             hipStream_t stream);
// Tiling of a batched projection: token groups per block (tg: 1, 2, 4, 8),
// row blocks per wave (rbw) and column splits (nsplit), chosen so the grid
// fills the chip with the fewest re-decodes of the weights.
struct MatmulPlan {
    int tg, rbw, nsplit;
};
// hl: operands as high + low fp16 parts (the model's prefill).
MatmulPlan hexmm_plan(int M, int rows, int cols, bool hl = false);
hipError_t launch_hexmm(const MatmulArgs& a, hipStream_t stream);
// tmp[m][j] = S[j] * sum_c bf16(X[m][c]) * Vt[j][c]
hipError_t launch_lowrank_batched(const uint16_t* X, const uint16_t* Vt, const float* S, float* tmp,
                                  int M, int k, int cols, hipStream_t stream);
hipError_t launch_lowrank(const float* x, const uint16_t* Vt, const float* S, float* tmp_k,
                          int k, int cols, hipStream_t stream);
hipError_t launch_rmsnorm(const float* x, const float* w, float* out, int dim, float eps,
                          hipStream_t stream);
hipError_t launch_vec_add(float* y, const float* a, const float* b, int dim, hipStream_t stream);
hipError_t launch_swiglu(const float* g, const float* u, float* out, int dim, hipStream_t stream);
hipError_t launch_rope_kv(float* q, const float* k, const float* v, const RopeKV& r,
                          const float2* cs_inline, hipStream_t stream);
// The same for M consecutive tokens: q [M][n_heads*hd] in place, k / v
// [M][n_kv*hd], token m at position r.pos + m (r.cs holds every position).
hipError_t launch_rope_kv_rows(float* q, const float* k, const float* v, const RopeKV& r, int M,
                               hipStream_t stream);

// Contexts up to this length run attention as one block per KV head (the
// score buffer of attn_kernel holds 256 positions).
constexpr int kShortCtx = 256;
// the decode graphs of short contexts: one attention chunk per KV head, sized
// to the position (a chunk's rows are loaded whatever the position)
constexpr int kShortTiers = 3;
constexpr int kShortChunk[kShortTiers] = {64, 128, kShortCtx};

struct AttnArgs {
    const float* q;
    const uint16_t* k_cache;
    const uint16_t* v_cache;
    float* out;
    const int* pos_dev;   // null -> pos
    int pos;
    int layer, n_heads, n_kv, hd, max_seq;
    float sm_scale;
    int chunk;            // positions per split
    int max_splits;       // grid.y
    // Splits of a KV head hand their partials (max, sum, o[hd] per query
    // head) to the block of the last split as 64-bit words, epoch << 32 |
    // float bits, one relaxed device-scope store each: a word read with the
    // launch's epoch is that launch's value, so there is no fence and no
    // clearing.  Epoch source: `epoch` when nonzero (chosen by the host,
    // different for every launch on a workspace: words left by launches of
    // another shape then never match), else counters[kvh], the head's launch
    // count (the epoch is the count + 1, advanced by the merging block; for
    // graph replays of one shape).  Zero ws and counters at allocation.
    unsigned long long* ws;   // [n_kv][max_splits][group][2 + hd]
    unsigned* counters;       // [n_kv] (epoch == 0 and dep == null only)
    unsigned* err;            // set to 1 when a wait for a partial runs out (may be null)
    unsigned epoch;
    // Third epoch source (epoch == 0, counters == null; one-token launches
    // with a host position): device words dep[0] = the epoch of the last
    // launch on the workspace (low half), dep[2] = KV heads merged in this
    // launch.  Every block reads dep[0] at its start and tags its words with
    // the next epoch (0 skipped); the merging block of each KV head's last
    // split, once every split's words are in (so every block of the head has
    // read dep[0]), adds one to dep[2], and the last head to do so clears
    // dep[2] and stores the new epoch.  Each launch thus takes a new epoch on
    // the device, also when a captured graph replays it, and words of earlier
    // launches of any shape never match.  n_kv atomics per launch: one per
    // block on a single word (an arrival count) serialised for microseconds.
    // Zero at allocation.
    unsigned long long* dep;
    // merging blocks: polling rounds before a wait counts as timed out
    // (0: the default bound)
    int spin_limit;
    // test only (0 in use): merging blocks wait for the tag epoch +
    // wait_skew, which no split writes, so the bounded wait runs out and
    // sets *err while every block still finishes
    int wait_skew;
    // one-token matrix-core kernel: blocks that merge a KV head's splits
    // (0 or 1: the last split's; up to 8 when every block of the grid is
    // resident at once; set by the launcher)
    int mergers;
};
hipError_t launch_attention(const AttnArgs& a, hipStream_t stream);
// Causal attention of M consecutive prompt tokens on the matrix cores:
// token t (query rows q[t][n_heads][hd], RoPE applied; its K/V rows already
// in the cache at p0 + t) over cache positions 0 .. p0 + t, out[t][n_heads][hd].
// Group sizes 1, 2, 4, 8; head dims 64, 128, 256; p0 + M <= max_seq.  No
// workspace, no waits between blocks.
struct PrefillAttn {
    const float* q;
    const uint16_t* k_cache;
    const uint16_t* v_cache;
    float* out;
    int layer, p0, M, n_heads, n_kv, hd, max_seq;
    float sm_scale;
    int log2g;   // set by the launcher
};
hipError_t launch_prefill_attention(const PrefillAttn& a, hipStream_t stream);
// RoPE + K/V append at a.pos fused into the one-token attention launch
// (host position; k, v: the new rows before RoPE; cs: (cos, sin) of pos,
// hd / 2 pairs): q is rotated in place, the cache rows written, out as
// launch_attention.  hipErrorNotSupported for shapes the fused kernel does
// not cover (then run launch_rope_kv and launch_attention).
hipError_t launch_rope_attention(const AttnArgs& a, const float* k, const float* v, int interleaved,
                                 const float2* cs, hipStream_t stream);
// Polling rounds of a merging block (each ~50 ns of s_sleep plus a round
// trip; about 0.2 s in all) before its wait counts as timed out.
constexpr int kAttnSpinLimit = 1 << 22;
// Positions per attention split for a context of n_ctx positions: one
// split up to 128 positions (no hand-over, no merge; the shortest chunk
// that holds them: fewer positions per wave); beyond, enough splits to
// spread the context over the chip (n_kv * splits ~ 256 blocks), 64, 128 or
// 256 positions each (256 is the kernels' LDS score buffer).
inline int attention_chunk(int n_ctx, int n_kv) {
    if (n_ctx <= 128) return n_ctx <= 64 ? 64 : 128;
    const int want = (n_ctx * n_kv + 255) / 256;
    return want <= 64 ? 64 : (want <= 128 ? 128 : 256);
}
// Sets the calling thread's error text (gsdh_last_error) and returns code,
// or -1 for code 0.
int fail(int code, const char* fmt, ...);
size_t attention_ws_bytes(int n_kv, int max_splits, int group, int hd);
// Workspace of a stand-alone one-token attention launch (the operator
// twins): a 256-byte header (AttnArgs::dep: the epoch word at byte 0 and the
// head count at byte 16; the error word at byte 8), then the split words.
// Zero at allocation; never cleared after.
constexpr size_t kAttnWsHeader = 256;
// Split words a workspace must hold for every context of 1 .. max_ctx
// positions (the chunking of attention_chunk), header excluded.
size_t attention_ws_bytes_upto(int n_kv, int group, int hd, int max_ctx);
// Fills the epoch, workspace and error fields of a one-token attention
// launch from a workspace laid out as above (splits > 1 only: a single split
// hands nothing over).
inline void attention_use_ws(AttnArgs& a, unsigned long long* hdr) {
    a.epoch = 0;
    a.counters = nullptr;
    a.dep = a.max_splits > 1 ? hdr : nullptr;
    a.err = reinterpret_cast<unsigned*>(hdr + 1);
    a.ws = hdr + kAttnWsHeader / 8;
}
// The library's static scratch of the current device (gsd_noalloc.hip) as a
// one-token launch's workspace (a.n_kv, a.hd and a.max_splits set); fails
// when the partials do not fit it.
int attention_static_ws(hipStream_t stream, AttnArgs& a, int group, const char* who);
// After a synchronisation: whether a merge's wait on the static scratch ran
// out since the last check (the word is cleared).
int attention_static_error(int* was_set);
// Test-only settings of the stand-alone attention launches, read from the
// environment at each call (GSD_ATTN_TEST_SKEW -> wait_skew,
// GSD_ATTN_SPIN_LIMIT -> spin_limit); both unset in use.
void attention_test_knobs(AttnArgs& a);

// embedding row of *token_dev to fp32 x; also zeroes clear[0..nclear) (the
// rank-k publication words of the token's matvec launches) and, when epoch
// is non-null, advances the token counter *epoch by one
hipError_t launch_embed(const uint16_t* embed, const int* token_dev, float* x, int hidden,
                        unsigned long long* clear, int nclear, unsigned* epoch, hipStream_t stream);

// Greedy argmax with the reference's nan_to_num (gsd_lq_cpu_runtime.py:423);
// with a step state st it writes the token and the margin top1-top2 there
// and, when gen_tokens != null, appends both to the gen arrays at
// st->gen_count (advance: st->pos += 1); with st == null it writes them to
// gen_tokens[0] and gen_margins[0] only.
struct StepState {
    int token;
    int pos;
    int gen_count;
    int margin_bits;    // top1 - top2 of the last argmax (float bits)
    unsigned err;       // nonzero: a bounded in-kernel wait timed out
    int pad[3];
};
// words (3 kArgBlocks) and ctr (kArgBlocks, zero at first use, used by one
// launch at a time): the multi-block form; otherwise one block
constexpr int kArgBlocks = 32;
hipError_t launch_argmax(const float* logits, int n, StepState* st, int* gen_tokens,
                         float* gen_margins, int advance, hipStream_t stream,
                         unsigned long long* words = nullptr, unsigned* ctr = nullptr);
// st->token, pos = (token, pos), gen_count = 0; err cleared only with reset_err
hipError_t launch_set_step(StepState* st, int token, int pos, int reset_err, hipStream_t stream);
hipError_t launch_fill_u32(unsigned* p, unsigned v, size_t n, hipStream_t stream);
hipError_t launch_unpack(const uint8_t* codes, int64_t n, int radius, int32_t* idx,
                         int8_t* r01, hipStream_t stream);

hipError_t launch_copy(const void* src, void* dst, size_t nbytes, hipStream_t stream);
// codes of a tensor's tiled layout back in file order (u8 [rows][cols / 2], device)
hipError_t launch_tile_codes(const HexSeg& s, int cols, uint8_t* out, hipStream_t stream);

int device_cu_count();

}  // namespace gsd
