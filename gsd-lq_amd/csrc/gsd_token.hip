// gsd_token.hip -- the persistent token kernel: a whole decode step (the
// reference's per-token sequence, run_gpu_native_chat.py:892-969, with the
// engine arithmetic of gsd_lq_cpu_engine.c) in one launch of one 512-thread
// block per CU.
//
// Why one launch: a token is ~5 dependent phases per layer.  As separate
// launches each phase pays dispatch, a prologue (input vector, norm
// statistics, codebook copies, first weight loads) and a drain tail, a few
// microseconds of idle HBM each.  Here the blocks stay resident, the codebook
// is copied into LDS once per token, and every projection phase issues its
// first weight loads before it waits for its input vector, so the weight
// stream of the next phase is already in flight while the previous phase's
// last rows are produced.
//
// Hand-off between phases: every element of an intermediate vector (q, k, v,
// attention output, residual stream, SwiGLU output, attention partials,
// per-block top-2) is one 64-bit word  epoch << 32 | float bits,  written
// with a single device-scope store and read with device-coherent loads
// (16-byte buffer loads with sc1; the two 8-byte halves are separate words).
// A reader takes a word once it carries the launch's epoch.  Each vector has
// its own slot per layer and is written once per launch, and the epoch is a
// per-block launch counter that every block advances at its end, so nothing
// is ever cleared and no fence or grid barrier is used.  All waits are
// bounded by a 20 ms clock limit; one that runs out sets StepState::err,
// after which later waits give up at once and the launch drains.
//
// Work split per projection phase: units of 16 rows (gate/up: 16 rows of
// each) go to block u mod grid; within a block the waves split the 128-column
// chunks of a unit exactly as the stand-alone MFMA matvec does (the same
// lattice-form v_mfma_f32_16x16x32_f16 step, per-row scale, fp32 partials
// summed in the same order), so the rows equal that kernel's.  Attention runs
// one item per (query head, 256-position split) on the last blocks of the
// grid; splits publish (max, sum, o) partials and the first blocks merge them.
#include <algorithm>

#include "gsd_internal.h"
#include "gsd_device.h"

namespace gsd {

TokWords tok_words(int hidden, int ffn, int n_heads, int n_kv, int hd, int max_seq) {
    TokWords w{};
    const int qd = n_heads * hd, kvd = n_kv * hd;
    const int smax = (max_seq + kTokChunk - 1) / kTokChunk;
    w.q = 0;
    w.k = w.q + qd;
    w.v = w.k + kvd;
    w.att = w.v + kvd;
    w.mid = w.att + qd;
    w.h = w.mid + hidden;
    w.x = w.h + ffn;
    w.part = w.x + hidden;
    w.total = w.part + (smax > 1 ? n_heads * smax * (2 + hd) : 0);
    w.total = (w.total + 1) & ~1;   // every vector starts 16-byte aligned
    return w;
}

namespace {

typedef unsigned long long u64;
// Arguments, layer table and segment descriptors are read through the
// constant address space: uniform reads become scalar loads.
#define AS4 __attribute__((address_space(4)))
typedef const AS4 TokArgs CArgs;
typedef const AS4 HexSeg CSeg;
typedef const AS4 TokLayer CLayer;
constexpr int kTokWaves = kTokThreads / 64;
constexpr int kTokJ = kTokMaxCols / (2 * kTokThreads);   // input pairs per thread
constexpr int kTokXBytes = kTokMaxCols / 128 * 512;       // A-operand staging
constexpr u64 kWaitTicks = 2000000ull;                    // 20 ms of the 100 MHz clock
constexpr int kEpiHead = 4;                               // logits + running top-2
constexpr int kRing = 8;                                  // chunk loads in flight per wave
constexpr int kRedSlots = 2 * kRing;                      // unit partial-sum slots (power of two)
constexpr int kStageUnits = 8;                            // units per block whose epilogue inputs are staged
constexpr int kStageRank = 2;                             // rank-k terms staged per row
constexpr int kStageKinks = 4;                            // kinks staged per row
constexpr int kRkRegs = 28;                               // rank-k row words prefetched per thread

#define AS1 __attribute__((address_space(1)))
__device__ __forceinline__ void publish(u64* p, unsigned ep, float v) {
    __hip_atomic_store((AS1 u64*)p, ((u64)ep << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 peek(const u64* p) {
    return __hip_atomic_load((AS1 u64*)const_cast<u64*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One more round of a bounded wait, or false once the caller must give up
// (the limit ran out now or in an earlier wait of the launch).
__device__ bool wait_more(u64& t0, int tries, unsigned* err) {
    if (tries == 0) {
        if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) return false;
        t0 = __builtin_amdgcn_s_memrealtime();
    } else if (__builtin_amdgcn_s_memrealtime() - t0 > kWaitTicks) {
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    __builtin_amdgcn_s_sleep(2);
    return true;
}

// value of word *p: w is a load of it already made; waits if it is stale
__device__ __forceinline__ float word_val(u64 w, const u64* p, unsigned ep, unsigned* err) {
    if ((unsigned)(w >> 32) != ep) {
        u64 t0 = 0;
        for (int tries = 0; (unsigned)((w = peek(p)) >> 32) != ep; tries++)
            if (!wait_more(t0, tries, err)) break;
    }
    return __uint_as_float((unsigned)w);
}
__device__ __forceinline__ float take(const u64* p, unsigned ep, unsigned* err) {
    return word_val(peek(p), p, ep, err);
}

// Position of pair p (columns 2p, 2p + 1) in the A-operand staging: chunk
// c = p / 64 holds 32 16-byte rows [h][t][g][hi/lo]; the pair's fp16 (u, v)
// hi part is the u32 at the returned index, its lo part 4 u32 further on.
__device__ __forceinline__ int xslot(int p) {
    const int c = p >> 6, h = (p >> 5) & 1, g = (p >> 3) & 3, t = (p >> 2) & 1, e = p & 3;
    return ((((c * 2 + h) * 2 + t) * 4 + g) * 2) * 4 + e;
}

template <int TB>
struct TokSmem {
    uint32_t stab[TB * 64];                          // codebook: entry e of lane l at byte 256 e + 4 l
    float red[kRedSlots][kTokWaves][16];             // per-wave row partials of a unit
    unsigned cnt[kRedSlots];                         // partials deposited in a slot (cumulative)
    unsigned done[kRedSlots];                        // units of a slot finalized (cumulative)
    unsigned rdy;                                    // waves whose epilogue inputs are in LDS
    float scr[2][kTokWaves];                         // norm statistics
    float tks[kTokWaves][kMaxSeg * kMaxRank];        // rank-k partials
    // epilogue inputs of the block's first kStageUnits units, entry
    // e = (unit * 2 + group) * 16 + row: residual input, U row, kinks
    float pres[kStageUnits * 16];
    uint32_t ustg[kStageUnits * 2 * 16];             // U row (k <= kStageRank) as fp16 pair
    int nkin[kStageUnits * 2 * 16];
    int kcol[kStageUnits * 2 * 16][kStageKinks];
    float kdl[kStageUnits * 2 * 16][kStageKinks];
    Top2 tops[kTokWaves];
};

// One projection phase.  Its segments are consecutive in the layer table
// (q, k, v / gate, up), and with kEpiStore their outputs are consecutive
// vectors of words (q, k, v), so both are addressed by offset, not by
// selecting among fields.
struct LinDesc {
    CSeg* s0;
    int nseg, epi, cols;
    const u64* in;          // input words; null: the token's embedding row
    const float* norm_w;    // null: no RMSNorm
    u64* out;               // output words (kEpiStore: segment g's rows follow segment g-1's)
    const u64* resid;       // kEpiResidual input words; null: the embedding row
};

// Lane id re-derived (from the exec mask count, not the work-item id) and
// made opaque at each phase start: otherwise the compiler hoists every
// per-thread index of every phase out of the token's phase loop and keeps
// them all live (spilled) for the whole launch.
__device__ __forceinline__ int phase_lane() {
    int lane = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    __asm__ volatile("" : "+v"(lane));
    return lane;
}
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

template <int TB>
__device__ __forceinline__ void lin_phase(CArgs* a, const LinDesc& D, TokSmem<TB>& sm, uint4* X,
                                          unsigned ep, int token, int& rbuf, Top2& top, int wid) {
    const int lane = phase_lane(), tid = wid * 64 + lane;
    const int nblk = (int)gridDim.x, b = (int)blockIdx.x;
    unsigned* err = &a->st->err;
    const int nc = (D.cols + 127) >> 7;
    const bool paired = D.epi == kEpiSwiGLU;
    const int G = paired ? 2 : 1, WG = kTokWaves / G;
    int WR = WG;   // waves per unit: a power of two dividing nc
    while (nc % WR) WR >>= 1;
    const int grp = wid / WG, wr = wid - grp * WG;
    const bool active = wr < WR;
    CSeg* S0 = D.s0;
    CSeg* S1 = D.s0 + (D.nseg > 1 ? 1 : 0);
    CSeg* S2 = D.s0 + (D.nseg > 2 ? 2 : 0);
    const int nrb0 = (S0->rows + 15) >> 4;
    const int ub1 = nrb0, ub2 = ub1 + (D.nseg > 1 ? (S1->rows + 15) >> 4 : 0);
    const int ub3 = ub2 + (D.nseg > 2 ? (S2->rows + 15) >> 4 : 0);
    const int nunits = paired ? nrb0 : ub3;
    auto seg_of = [&](int u) { return paired ? grp : (u >= ub2 ? 2 : (u >= ub1 ? 1 : 0)); };
    auto segp = [&](int g) { return D.s0 + g; };
    auto ubase = [&](int g) { return g == 0 ? 0 : (g == 1 ? ub1 : ub2); };
    const int P = nc / WR;
    const int my_units = b < nunits ? (nunits - 1 - b) / nblk + 1 : 0;
    const int nsteps = active ? P * my_units : 0;   // steps of this wave

    // weight ring: kRing chunk loads in flight per wave, the first ones issued
    // before the input vector is waited for (the cursor clamps to the last
    // unit, so loads past a wave's last step stay in bounds)
    // code tiles: 7-bit for codebooks of at most 128 points
    constexpr bool kB7 = TB <= 128;
    constexpr int kTileB = kB7 ? kTile7 : kTileU8;
    const uint32_t lof = tile_lane_off(kB7, lane);
    int lk = 0, lj = 0;
    const unsigned char* lcb = nullptr;
    const uint32_t* lsb = nullptr;
    auto lset = [&](int k) {
        const int uu = min(b + k * nblk, nunits - 1);
        const int g = seg_of(uu);
        const int rb = paired ? uu : uu - ubase(g);
        CSeg* sg = segp(g);
        lcb = reinterpret_cast<const unsigned char*>(sg->codes_t) + (size_t)rb * nc * kTileB;
        lsb = sg->scales_t + (size_t)rb * nc * 16;
    };
    const int wrl = active ? wr : 0;   // inactive waves load (and drop) in-bounds chunks
    auto lissue = [&](uint4& cw, uint32_t& sw) {
        const int c = wrl + lj * WR;
        cw = tile_load(lcb + (size_t)c * kTileB + lof);
        sw = lsb[c * 16 + (lane & 15)];
        if (++lj == P) {
            lj = 0;
            lset(++lk);
        }
    };
    // Loads go out in the order their data is needed back (completion is in
    // issue order): norm weights, the input words (the wait), then half the
    // weight ring (HBM), which lands during the wait; the epilogue inputs,
    // rank-k rows and the other ring half follow the second barrier.

    // norm weights of the thread's first two pairs (all of them for inputs of
    // up to 4096 columns)
    constexpr float kS32 = 0.866025403784438646763723170752936183f;
    uint32_t* X32 = reinterpret_cast<uint32_t*>(X);
    const int jn = (D.cols + 2 * kTokThreads - 1) / (2 * kTokThreads);
    const float2* nw2 = reinterpret_cast<const float2*>(D.norm_w);
    float2 nwa = make_float2(1.f, 1.f), nwb = nwa;
    if (nw2) {
        if (2 * tid < D.cols) nwa = nw2[tid];
        if (2 * (tid + kTokThreads) < D.cols) nwb = nw2[tid + kTokThreads];
    }

    // Rank-k rows: tmp[j] = S[j] * sum_c x'[c] Vt[j][c] (gsd_lq_cpu_engine.c:110-127)
    // over the terms of all segments.  Thread t takes items t + 512 i of the
    // flattened (term, pair) space; when the pair count is a multiple of 512,
    // item i is term i / npb at pair t + 512 (i mod npb) (npb = pairs / 512),
    // a pair this thread parks itself, and a wave's lanes share the term.
    int ntk = 0;
    for (int g = 0; g < D.nseg; g++) ntk += segp(g)->k;
    const int npairs = D.cols >> 1, npb = npairs / kTokThreads;
    const bool rk_fast = ntk > 0 && npairs % kTokThreads == 0 && ntk * npb <= kRkRegs;
    auto vt_row = [&](int idx) {
        int g = 0, jj = idx;
        while (jj >= segp(g)->k) {
            jj -= segp(g)->k;
            g++;
        }
        return reinterpret_cast<const uint32_t*>(segp(g)->Vt + (size_t)jj * D.cols);
    };
    // input words, then the ring
    u32x4v w[kTokJ];
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<u64*>(D.in), (short)0, D.in ? D.cols * 8 : 0, 0x00020000);
    auto issue_in = [&]() {
#pragma unroll
        for (int j = 0; j < kTokJ; j++)
            if (j < jn) w[j] = __builtin_amdgcn_raw_buffer_load_b128(r, (tid + j * kTokThreads) * 16, 0, 16 /* sc1 */);
    };
    if (D.in) issue_in();
    uint4 cr[kRing];
    uint32_t sr[kRing];
    lset(0);
#pragma unroll
    for (int i = 0; i < kRing / 2; i++) lissue(cr[i], sr[i]);

    // Input vector: pair p = tid + 512 j (columns 2p, 2p + 1) is read by this
    // thread only; x * w is parked in the two u32 of the pair's own A-operand
    // slot (no other thread touches them), so later passes need no barrier
    // between reading a pair and overwriting it with its operands.
    float ss = 0.f, mx = 0.f;
    auto park = [&](int j, int p, float xa, float xb) {   // stats of x and x * w
        const float2 w2 = j == 0 ? nwa : (j == 1 ? nwb : (nw2 ? nw2[p] : make_float2(1.f, 1.f)));
        ss = fmaf(xa, xa, ss);
        ss = fmaf(xb, xb, ss);
        const float p0 = xa * w2.x, p1 = xb * w2.y;
        mx = fmaxf(mx, fmaxf(fabsf(p0), fabsf(fmaf(kS32, p1, 0.5f * p0))));
        const int q = xslot(p);
        X32[q] = __float_as_uint(p0);
        X32[q + 4] = __float_as_uint(p1);
    };
    if (D.in) {
        u64 t0 = 0;
        for (int tries = 0;; tries++) {
            bool ok = true;
#pragma unroll
            for (int j = 0; j < kTokJ; j++)
                if (j < jn && 2 * (tid + j * kTokThreads) < D.cols && (w[j][1] != ep || w[j][3] != ep)) ok = false;
            if (ok || !wait_more(t0, tries, err)) break;
            issue_in();
        }
#pragma unroll
        for (int j = 0; j < kTokJ; j++) {
            const int p = tid + j * kTokThreads;
            if (j < jn && 2 * p < D.cols) park(j, p, __uint_as_float(w[j][0]), __uint_as_float(w[j][2]));
        }
    } else {
        const uint32_t* er = reinterpret_cast<const uint32_t*>(a->embed + (size_t)token * a->hidden);
        for (int j = 0; j < jn; j++) {
            const int p = tid + j * kTokThreads;
            if (2 * p < D.cols) {
                const uint32_t e2 = er[p];
                park(j, p, h2f((uint16_t)(e2 & 0xFFFFu)), h2f((uint16_t)(e2 >> 16)));
            }
        }
    }

    // sum x^2 and the largest |u|, |v| of x * w (gsd_lq_cpu_engine.c:66-82)
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        ss += __shfl_xor(ss, o, 64);
        mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    }
    if (lane == 0) {
        sm.scr[0][wid] = ss;
        sm.scr[1][wid] = mx;
    }
    lds_barrier();
    ss = 0.f;
    mx = 0.f;
    for (int w = 0; w < kTokWaves; w++) {
        ss += sm.scr[0][w];
        mx = fmaxf(mx, sm.scr[1][w]);
    }
    if (tid < kRedSlots) {
        sm.cnt[tid] = 0u;
        sm.done[tid] = 0u;
    }
    if (tid == 0) sm.rdy = 0u;
    const float inv = D.norm_w ? 1.0f / sqrtf(ss / (float)D.cols + a->eps) : 1.f;
    mx *= inv;
    int ex = 0;
    if (mx > 0.f && mx < INFINITY) (void)frexpf(mx, &ex);
    const float up = ldexpf(1.f, 14 - ex), down = ldexpf(1.f, ex - 14);

    // x' = (x * w) * inv as (u, v) * 2^e in fp16 hi / lo, in place of the parked pair
    auto put = [&](int p, float xa, float xb) {
        const float uu = xa * up, vv = fmaf(kS32, xb, 0.5f * xa) * up;
        const _Float16 uh = (_Float16)uu, vh = (_Float16)vv;
        const _Float16 ul = (_Float16)(uu - (float)uh), vl = (_Float16)(vv - (float)vh);
        const int q = xslot(p);
        X32[q] = (uint32_t)__builtin_bit_cast(uint16_t, uh) | ((uint32_t)__builtin_bit_cast(uint16_t, vh) << 16);
        X32[q + 4] = (uint32_t)__builtin_bit_cast(uint16_t, ul) | ((uint32_t)__builtin_bit_cast(uint16_t, vl) << 16);
    };
    for (int p = tid; p < npairs; p += kTokThreads) {
        const int q = xslot(p);
        put(p, __uint_as_float(X32[q]) * inv, __uint_as_float(X32[q + 4]) * inv);
    }
    for (int p = npairs + tid; p < nc * 64; p += kTokThreads) put(p, 0.f, 0.f);   // padding
    lds_barrier();

    // x' back from the staged operands: u = x'a 2^e, v = (x'a / 2 + s x'b) 2^e
    // as hi + lo fp16 (22 significant bits)
    auto xfull = [&](int p, float& xa, float& xb) {
        const int q = xslot(p);
        const uint32_t hi = X32[q], lo = X32[q + 4];
        xa = (h2f((uint16_t)(hi & 0xFFFFu)) + h2f((uint16_t)(lo & 0xFFFFu))) * down;
        const float v = (h2f((uint16_t)(hi >> 16)) + h2f((uint16_t)(lo >> 16))) * down;
        xb = (v - 0.5f * xa) * (1.0f / kS32);
    };
    // Epilogue inputs of the block's first kStageUnits units: thread
    // i < nstg * 16 G loads entry i (unit i / 16G, group, row) into registers,
    // with its rank-k rows, now that the first ring half has landed; both go
    // to LDS after the wave's first group of steps (stage_in), off the path
    // to the first step.  An epilogue waits until every wave has put its
    // share (rdy).
    const int nstg = min(my_units, kStageUnits);
    const int se = tid, sk = se / (16 * G), sgi_ = paired ? (se >> 4) % G : seg_of(b + sk * nblk);
    const bool sact = se < nstg * 16 * G;
    CSeg* ssg = segp(sact ? sgi_ : 0);
    const int su = b + sk * nblk;
    const int srow = (paired ? su : su - ubase(sgi_)) * 16 + (se & 15);
    const bool srow_ok = sact && srow < ssg->rows;
    // raw loads only: nothing computed on them before stage_in, so no lane
    // waits for them here
    u64 spw = 0ull;         // residual word
    uint32_t spe = 0u;      // or the embedding value (fp16 bits)
    uint32_t su0 = 0u, su1 = 0u, srp0 = 0u, srp1 = 0u;
    if (srow_ok) {
        if (D.epi == kEpiResidual) {
            if (D.resid) spw = peek(D.resid + srow);
            else spe = a->embed[(size_t)token * a->hidden + srow];
        }
        const int kk = ssg->k;
        if (kk > 0 && kk <= kStageRank) {
            su0 = ssg->U[(size_t)srow * kk];
            if (kk > 1) su1 = ssg->U[(size_t)srow * kk + 1];
        }
        if (ssg->row_ptr) {
            srp0 = ssg->row_ptr[srow];
            srp1 = ssg->row_ptr[srow + 1];
        }
    }

    // rank-k rows of this thread's items (term pointers advanced term by term)
    uint32_t vq[kRkRegs];
    {
        int tg = 0, tj = 0;   // segment, term within it
        while (tg < D.nseg && segp(tg)->k == 0) tg++;
        const uint32_t* vtp = rk_fast ? reinterpret_cast<const uint32_t*>(segp(tg)->Vt) : nullptr;
#pragma unroll
        for (int i = 0; i < kRkRegs; i++) {
            vq[i] = 0u;
            if (rk_fast && i < ntk * npb) {
                const int j = i % npb;
                if (i > 0 && j == 0) {   // next term
                    if (++tj == segp(tg)->k) {
                        tj = 0;
                        do tg++; while (segp(tg)->k == 0);
                        vtp = reinterpret_cast<const uint32_t*>(segp(tg)->Vt);
                    } else {
                        vtp += npairs;
                    }
                }
                vq[i] = vtp[tid + j * kTokThreads];
            }
        }
    }

    // the other half of the ring
#pragma unroll
    for (int i = kRing / 2; i < kRing; i++) lissue(cr[i], sr[i]);

    bool staged = false;
    auto stage_in = [&]() {
        if (sact) {
            const int e = (sk * 2 + (paired ? (se >> 4) % G : 0)) * 16 + (se & 15);
            if (D.epi == kEpiResidual && !paired)
                sm.pres[sk * 16 + (se & 15)] = !srow_ok ? 0.f : (D.resid ? word_val(spw, D.resid + srow, ep, err) : h2f((uint16_t)spe));
            sm.ustg[e] = su0 | (su1 << 16);
            const int nk = srow_ok && ssg->row_ptr ? (int)(srp1 - srp0) : 0;
            sm.nkin[e] = nk;
            for (int j = 0; j < min(nk, kStageKinks); j++) {
                sm.kcol[e][j] = ssg->kcols[srp0 + j];
                sm.kdl[e][j] = ssg->kdel[srp0 + j];
            }
        }
        // rank-k partial sums of x', per wave
        if (rk_fast) {
            float ar = 0.f;
    #pragma unroll
            for (int i = 0; i < kRkRegs; i++) {
                if (i < ntk * npb) {
                    const int idx = i / npb, j = i - idx * npb;
                    float xa, xb;
                    xfull(tid + j * kTokThreads, xa, xb);
                    ar = fmaf(xa, h2f((uint16_t)(vq[i] & 0xFFFFu)), ar);
                    ar = fmaf(xb, h2f((uint16_t)(vq[i] >> 16)), ar);
                    if (j == npb - 1) {
                        const float d = wave_sum(ar);
                        if (lane == 0) sm.tks[wid][idx] = d;
                        ar = 0.f;
                    }
                }
            }
        } else {
            for (int idx = 0; idx < ntk; idx++) {
                const uint32_t* vt = vt_row(idx);
                float d = 0.f;
                for (int p = tid; p < npairs; p += kTokThreads) {
                    float xa, xb;
                    xfull(p, xa, xb);
                    const uint32_t v2 = vt[p];
                    d = fmaf(xa, h2f((uint16_t)(v2 & 0xFFFFu)), d);
                    d = fmaf(xb, h2f((uint16_t)(v2 >> 16)), d);
                }
                d = wave_sum(d);
                if (lane == 0) sm.tks[wid][idx] = d;
            }
        }
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);
        if (lane == 0) (void)__hip_atomic_fetch_add(&sm.rdy, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        staged = true;
    };

    const uint32_t lane_off = (uint32_t)lane * 4u;
    const int m = lane & 15, lg = lane >> 4;
    const uint32_t sh7 = (uint32_t)(lane & 1) * 16u;
    auto step = [&](int c, const uint4 cw, const uint32_t sw, float& acc) {
        const unsigned char* tb = reinterpret_cast<const unsigned char*>(sm.stab);
        uint32_t w4[4] = {cw.x, cw.y, cw.z, cw.w};
        if constexpr (kB7) align7(w4, sh7);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint4 xq = X[(((c * 2 + h) * 2 + t) * 4 + lg) * 2 + (m & 1)];
                u32x4v aw;
                aw[0] = xq.x; aw[1] = xq.y; aw[2] = xq.z; aw[3] = xq.w;
                u32x4v bw;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t addr = code_addr(w4, 4 * (2 * h + t) + e, lane_off, kB7);
                    bw[e] = *reinterpret_cast<const uint32_t*>(tb + addr);
                }
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, aw), __builtin_bit_cast(half8v, bw),
                                                          d, 0, 0, 0);
            }
            const uint16_t sh = (uint16_t)(h ? (sw >> 16) : (sw & 0xFFFFu));
            acc = fmaf(d[0] + d[1], h2f(sh), acc);
        }
    };

    // x'[col] for the kink terms
    auto xnorm = [&](int col) {
        float xa, xb;
        xfull(col >> 1, xa, xb);
        return (col & 1) ? xb : xa;
    };

    // Unit completion without block barriers: each contributing wave deposits
    // its 16 row partials in the unit's slot and counts itself in; the wave
    // that arrives last finalizes the unit (after its current group of steps)
    // and marks the slot free.  Slot reuse waits for that mark; the wave that
    // owns the oldest pending unit never waits on a later one (kRedSlots >=
    // kRing), so the waits end.
    const int nwu = WR * G;
    auto arrive = [&](int k, float v) -> bool {
        const int slot = k & (kRedSlots - 1);
        const unsigned use = (unsigned)(k / kRedSlots);
        if (use > 0u) {
            u64 t0 = 0;
            for (int tries = 0; __hip_atomic_load(&sm.done[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < use; tries++)
                if (!wait_more(t0, tries, err)) break;
        }
        if (lane < 16) sm.red[slot][wid][lane] = v;
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);   // partials written before the count
        unsigned old = 0u;
        if (lane == 0) old = __hip_atomic_fetch_add(&sm.cnt[slot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        old = (unsigned)__builtin_amdgcn_readfirstlane((int)old);
        __asm__ volatile("" ::: "memory");
        return old == (use + 1u) * (unsigned)nwu - 1u;
    };
    bool inputs_in = false;
    auto finalize = [&](int k) {
        if (!inputs_in) {   // every wave's epilogue inputs are in LDS (normally long done)
            u64 t0 = 0;
            for (int tries = 0; __hip_atomic_load(&sm.rdy, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < (unsigned)kTokWaves; tries++)
                if (!wait_more(t0, tries, err)) break;
            inputs_in = true;
        }
        const int slot = k & (kRedSlots - 1);
        const int u = b + k * nblk;
        const int gu = paired ? 0 : seg_of(u);
        if (lane < 16) {
            float fin0 = 0.f, fin1 = 0.f;
#pragma unroll
            for (int gi = 0; gi < 2; gi++) {
                if (gi >= G) break;
                const int sgi = paired ? gi : gu;
                CSeg* sg = segp(sgi);
                const int row = (paired ? u : u - ubase(sgi)) * 16 + lane;
                float t = 0.f;
                for (int w = 0; w < WR; w++) t += sm.red[slot][gi * WG + w][lane];
                t *= down;
                if (row < sg->rows) {
                    const bool stg = k < kStageUnits;
                    const int e = (k * 2 + gi) * 16 + lane;
                    if (sg->row_ptr) {
                        const int nk = stg ? sm.nkin[e] : 0;
                        if (stg && nk <= kStageKinks) {
                            for (int i = 0; i < nk; i++) t += sm.kdl[e][i] * xnorm(sm.kcol[e][i]);
                        } else {
                            const uint32_t e1 = sg->row_ptr[row + 1];
                            for (uint32_t i = sg->row_ptr[row]; i < e1; i++) t += sg->kdel[i] * xnorm(sg->kcols[i]);
                        }
                    }
                    if (sg->k > 0) {
                        int off = 0;
                        for (int g2 = 0; g2 < sgi; g2++) off += segp(g2)->k;
                        const uint16_t* ur = sg->U + (size_t)row * sg->k;
                        for (int jj = 0; jj < sg->k; jj++) {
                            float tk = 0.f;
                            for (int w = 0; w < kTokWaves; w++) tk += sm.tks[w][off + jj];
                            const uint16_t uh = stg && sg->k <= kStageRank ? (uint16_t)(sm.ustg[e] >> (16 * jj)) : ur[jj];
                            t += h2f(uh) * (tk * sg->S[jj]);
                        }
                    }
                }
                if (gi == 0) fin0 = t;
                else fin1 = t;
            }
            CSeg* so = paired ? S0 : segp(gu);
            const int row = (paired ? u : u - ubase(gu)) * 16 + lane;
            if (row < so->rows) {
                if (paired) {
                    publish(D.out + row, ep, (fin0 / (1.0f + expf(-fin0))) * fin1);
                } else if (D.epi == kEpiStore) {
                    const int roff = (gu >= 1 ? S0->rows : 0) + (gu >= 2 ? S1->rows : 0);
                    publish(D.out + roff + row, ep, fin0);
                } else if (D.epi == kEpiResidual) {
                    const float pre = k < kStageUnits ? sm.pres[k * 16 + lane]
                                                      : (D.resid ? take(D.resid + row, ep, err)
                                                                 : h2f(a->embed[(size_t)token * a->hidden + row]));
                    publish(D.out + row, ep, pre + fin0);
                } else {
                    a->logits[row] = fin0;
                    top = merge(top, Top2{clean(fin0), -INFINITY, row});
                }
            }
        }
        __asm__ volatile("" ::: "memory");
        if (lane == 0)
            __hip_atomic_store(&sm.done[slot], (unsigned)(k / kRedSlots) + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };

    // steps in groups of kRing: step i of the group computes ring entry i and
    // reloads it with the step kRing ahead; units finalized by this wave are
    // handled after the group
    float acc = 0.f;
    int cj = 0, ck = 0;
    for (int s0 = 0; s0 < nsteps; s0 += kRing) {
        unsigned pend = 0u;
        const int pend_base = ck;
#pragma unroll
        for (int i = 0; i < kRing; i++) {
            if (s0 + i < nsteps) {
                step(wr + cj * WR, cr[i], sr[i], acc);
                lissue(cr[i], sr[i]);
                if (++cj == P) {
                    if (arrive(ck, acc)) pend |= 1u << (ck - pend_base);
                    acc = 0.f;
                    cj = 0;
                    ++ck;
                }
            }
        }
        if (!staged) stage_in();
        for (int j = 0; pend != 0u; j++, pend >>= 1)
            if (pend & 1u) finalize(pend_base + j);
    }
    if (!staged) stage_in();
}

// Attention of layer l at position pos (gsd_lq_cpu_engine.c:264-340 with the
// RoPE and KV append of :185-262): items (query head, 256-position split) on
// blocks grid-1, grid-2, ...; 16 waves cover the split's positions, LPP lanes
// per position.  The item holding position pos rotates the new k, rounds k
// and v to fp16, uses them from LDS and (first head of the KV group) appends
// them to the cache.
template <int HD>
__device__ __forceinline__ void attn_phase(CArgs* a, int l, int pos, unsigned ep, u64* W, float* sf, int wid) {
    constexpr int LPP = HD / 8, PPW = 64 / LPP, PPB = kTokWaves * PPW, UNR = kTokChunk / PPB;
    const int lane = phase_lane(), tid = wid * 64 + lane;
    const int nblk = (int)gridDim.x, b = (int)blockIdx.x;
    unsigned* err = &a->st->err;
    const int n = pos + 1, S = (n + kTokChunk - 1) / kTokChunk;
    const int nitems = a->n_heads * S, G = a->n_heads / a->n_kv;
    float* qr = sf;                                         // [HD] rotated q
    uint16_t* kn = reinterpret_cast<uint16_t*>(sf + HD);    // [HD] fp16 new k
    uint16_t* vn = kn + HD;                                 // [HD] fp16 new v
    float* sc = sf + 2 * HD;                                // [kTokChunk] scores
    float* part = sc + kTokChunk;                           // [waves][HD]
    float* ml = part + kTokWaves * HD;                      // max, sum
    const size_t rowstride = (size_t)a->n_kv * HD;
    const int sub = lane % LPP, prow = lane / LPP;

    for (int it = nblk - 1 - b; it < nitems; it += nblk) {
        const int h = it % a->n_heads, s = it / a->n_heads, kvh = h / G;
        const int t0 = s * kTokChunk, t1 = min(n, t0 + kTokChunk), cn = t1 - t0;
        const bool has_new = t1 == n;
        if (tid < HD) {
            const int d = tid;
            int d0, i;
            if (a->interleaved) {
                d0 = d & ~1;
                i = d >> 1;
            } else {
                i = d < HD / 2 ? d : d - HD / 2;
                d0 = i;
            }
            const int d1 = a->interleaved ? d0 + 1 : d0 + HD / 2;
            const float2 cs = a->cs[(size_t)pos * (HD / 2) + i];
            const u64* qw = W + a->wo.q + (size_t)h * HD;
            const u64* kw = W + a->wo.k + (size_t)kvh * HD;
            const u64* vw = W + a->wo.v + (size_t)kvh * HD;
            const u64 wq0 = peek(qw + d0), wq1 = peek(qw + d1);
            u64 wk0 = 0ull, wk1 = 0ull, wv0 = 0ull;
            if (has_new) {
                wk0 = peek(kw + d0);
                wk1 = peek(kw + d1);
                wv0 = peek(vw + d);
            }
            const float x0 = word_val(wq0, qw + d0, ep, err), x1 = word_val(wq1, qw + d1, ep, err);
            {
#pragma clang fp contract(off)
                qr[d] = d == d0 ? x0 * cs.x - x1 * cs.y : x0 * cs.y + x1 * cs.x;
            }
            if (has_new) {
                const float k0 = word_val(wk0, kw + d0, ep, err), k1 = word_val(wk1, kw + d1, ep, err);
                float ky;
                {
#pragma clang fp contract(off)
                    ky = d == d0 ? k0 * cs.x - k1 * cs.y : k0 * cs.y + k1 * cs.x;
                }
                const uint16_t kh = f2h(ky), vh = f2h(word_val(wv0, vw + d, ep, err));
                kn[d] = kh;
                vn[d] = vh;
                if (h % G == 0) {
                    const size_t at = ((size_t)l * a->max_seq + (size_t)pos) * rowstride + (size_t)kvh * HD + d;
                    a->k_cache[at] = kh;
                    a->v_cache[at] = vh;
                }
            }
        }
        lds_barrier();
        float qv[8];
#pragma unroll
        for (int e = 0; e < 8; e++) qv[e] = qr[sub * 8 + e];
        const uint16_t* kb = a->k_cache + (size_t)l * a->max_seq * rowstride + (size_t)kvh * HD + sub * 8;
        const uint16_t* vb = a->v_cache + (size_t)l * a->max_seq * rowstride + (size_t)kvh * HD + sub * 8;
        const int nst = (cn + PPB - 1) / PPB;   // <= UNR

        // scores s[t] = (q . K_t) * sm_scale
        uint4 kq[UNR];
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int t = min(t0 + u * PPB + wid * PPW + prow, t1 - 1);
            kq[u] = u < nst ? *reinterpret_cast<const uint4*>(kb + (size_t)t * rowstride) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            if (u < nst) {
                const int tl = u * PPB + wid * PPW + prow;
                const uint4 kk = (has_new && t0 + tl == pos) ? *reinterpret_cast<const uint4*>(kn + sub * 8) : kq[u];
                float kf[8];
                unpack8(kk, kf);
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++) d = fmaf(qv[e], kf[e], d);
                d = lane_group_sum<LPP>(d);
                if (sub == 0 && tl < cn) sc[tl] = d * a->sm_scale;
            }
        }
        lds_barrier();
        if (wid == 0) {
            float mm = -INFINITY;
            for (int i = lane; i < cn; i += 64) mm = fmaxf(mm, sc[i]);
            mm = wave_allmax(mm);
            float ll = 0.f;
            for (int i = lane; i < cn; i += 64) {
                const float e = expf(sc[i] - mm);
                sc[i] = e;
                ll += e;
            }
            ll = wave_allsum(ll);
            if (lane == 0) {
                ml[0] = mm;
                ml[1] = ll;
            }
        }
        lds_barrier();
        // o[d] = sum_t p[t] V_t[d]
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = 0.f;
        uint4 vq[UNR];
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int t = min(t0 + u * PPB + wid * PPW + prow, t1 - 1);
            vq[u] = u < nst ? *reinterpret_cast<const uint4*>(vb + (size_t)t * rowstride) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int tl = u * PPB + wid * PPW + prow;
            if (u < nst && tl < cn) {
                const uint4 vv = (has_new && t0 + tl == pos) ? *reinterpret_cast<const uint4*>(vn + sub * 8) : vq[u];
                float vf[8];
                unpack8(vv, vf);
                const float p = sc[tl];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[e] = fmaf(p, vf[e], acc[e]);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = slot_sum<LPP>(acc[e]);
        if (prow == 0) {
#pragma unroll
            for (int e = 0; e < 8; e++) part[wid * HD + sub * 8 + e] = acc[e];
        }
        lds_barrier();
        if (tid < HD) {
            float o = 0.f;
            for (int w = 0; w < kTokWaves; w++) o += part[w * HD + tid];
            if (S == 1) {
                publish(W + a->wo.att + (size_t)h * HD + tid, ep, o * (1.0f / ml[1]));
            } else {
                u64* pw = W + a->wo.part + ((size_t)h * S + s) * (2 + HD);
                publish(pw + 2 + tid, ep, o);
                if (tid < 2) publish(pw + tid, ep, ml[tid]);
            }
        }
        lds_barrier();   // the next item rewrites qr / kn / sc / part
    }
    // merge of the split partials of head h on block h mod grid
    if (S > 1) {
        for (int h = b; h < a->n_heads; h += nblk) {
            if (tid < HD) {
                const u64* base = W + a->wo.part + (size_t)h * S * (2 + HD);
                float M = -INFINITY;
                for (int sp = 0; sp < S; sp++) M = fmaxf(M, take(base + (size_t)sp * (2 + HD), ep, err));
                float L = 0.f, O = 0.f;
                for (int sp = 0; sp < S; sp++) {
                    const u64* pp = base + (size_t)sp * (2 + HD);
                    const u64 w0 = peek(pp), w1 = peek(pp + 1), w2 = peek(pp + 2 + tid);
                    const float f = expf(word_val(w0, pp, ep, err) - M);
                    L = fmaf(word_val(w1, pp + 1, ep, err), f, L);
                    O = fmaf(word_val(w2, pp + 2 + tid, ep, err), f, O);
                }
                publish(W + a->wo.att + (size_t)h * HD + tid, ep, O / L);
            }
        }
    }
}

// The arguments stay in the kernarg segment and are re-read through an
// opaque pointer at each phase, so they occupy registers only while a phase
// uses them.
__device__ __forceinline__ CArgs* args_ptr() {
    CArgs* p = (CArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    __asm__ volatile("" : "+s"(p));
    return p;
}

template <int TB, int HD>
__global__ void __launch_bounds__(kTokThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) tok_kernel(const TokArgs args, int with_head) {
    __shared__ TokSmem<TB> sm;
    __shared__ uint4 Xs[kTokXBytes / 16];
    const int wid = wave_id();
    const int b = (int)blockIdx.x, nblk = (int)gridDim.x;
    CArgs* a0 = args_ptr();
    unsigned ep = a0->epoch[b] + 1u;
    if (ep == 0u) ep = 1u;   // words start at 0: epoch 0 is never valid
    const int token = a0->st->token, pos = a0->st->pos;
    {
        const int lane = phase_lane();
        for (int e = wid; e < TB; e += kTokWaves) sm.stab[e * 64 + lane] = a0->fields[e];
    }

    int rbuf = 0;
    Top2 top{-INFINITY, -INFINITY, 0x7FFFFFFF};
    const int nph = a0->n_layers * 5 + (with_head ? 1 : 0);
    for (int ph = 0; ph < nph; ph++) {
        CArgs* a = args_ptr();
        const int l = ph / 5, k = ph - 5 * l;
        u64* W = a->words + (size_t)l * a->wo.total;
        const u64* xin = l > 0 ? a->words + (size_t)(l - 1) * a->wo.total + a->wo.x : nullptr;
        if (l < a->n_layers && k == 1) {
            attn_phase<HD>(a, l, pos, ep, W, reinterpret_cast<float*>(Xs), wid);
            continue;
        }
        LinDesc D;
        D.resid = nullptr;
        D.norm_w = nullptr;
        D.out = nullptr;
        if (l == a->n_layers) {   // final norm + lm_head
            D.s0 = (CSeg*)a->head; D.nseg = 1; D.epi = kEpiHead; D.in = xin; D.cols = a->hidden; D.norm_w = a->out_norm;
        } else {
            CLayer* L = (CLayer*)(a->layers + l);
            if (k == 0) {          // q, k, v with the attention RMSNorm (words q | k | v consecutive)
                D.s0 = &L->w[0]; D.nseg = 3; D.epi = kEpiStore;
                D.in = xin; D.cols = a->hidden; D.norm_w = L->norm[0]; D.out = W + a->wo.q;
            } else if (k == 2) {   // o + residual
                D.s0 = &L->w[3]; D.nseg = 1; D.epi = kEpiResidual; D.in = W + a->wo.att;
                D.cols = a->n_heads * a->hd; D.out = W + a->wo.mid; D.resid = xin;
            } else if (k == 3) {   // gate / up with the FFN RMSNorm, SwiGLU
                D.s0 = &L->w[4]; D.nseg = 2; D.epi = kEpiSwiGLU; D.in = W + a->wo.mid;
                D.cols = a->hidden; D.norm_w = L->norm[1]; D.out = W + a->wo.h;
            } else {               // down + residual
                D.s0 = &L->w[6]; D.nseg = 1; D.epi = kEpiResidual; D.in = W + a->wo.h; D.cols = a->ffn;
                D.out = W + a->wo.x; D.resid = W + a->wo.mid;
            }
        }
        lin_phase<TB>(a, D, sm, Xs, ep, token, rbuf, top, wid);
    }

    CArgs* a = args_ptr();
    const int lane = phase_lane(), tid = wid * 64 + lane;
    if (with_head) {
        // this block's top-2 (lanes 0..15 of every wave that finalized head
        // rows), then block 0 merges every block's and advances the step
        // state like argmax_kernel
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) {
            Top2 u{__shfl_xor(top.v1, o, 64), __shfl_xor(top.v2, o, 64), __shfl_xor(top.i1, o, 64)};
            top = merge(top, u);
        }
        if (lane == 0) sm.tops[wid] = top;
        __syncthreads();
        if (tid == 0) {
            Top2 r = sm.tops[0];
            for (int w = 1; w < kTokWaves; w++) r = merge(r, sm.tops[w]);
            u64* tw = a->top + (size_t)b * 4;
            publish(tw, ep, r.v1);
            publish(tw + 1, ep, __int_as_float(r.i1));
            publish(tw + 2, ep, r.v2);
        }
        __syncthreads();
        if (b == 0) {
            unsigned* err = &a->st->err;
            Top2 t{-INFINITY, -INFINITY, 0x7FFFFFFF};
            for (int i = tid; i < nblk; i += kTokThreads) {
                const u64* tw = a->top + (size_t)i * 4;
                const u64 w0 = peek(tw), w1 = peek(tw + 1), w2 = peek(tw + 2);
                Top2 u{word_val(w0, tw, ep, err), word_val(w2, tw + 2, ep, err),
                       __float_as_int(word_val(w1, tw + 1, ep, err))};
                t = merge(t, u);
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                Top2 u{__shfl_xor(t.v1, o, 64), __shfl_xor(t.v2, o, 64), __shfl_xor(t.i1, o, 64)};
                t = merge(t, u);
            }
            if (lane == 0) sm.tops[wid] = t;
            __syncthreads();
            if (tid == 0) {
                Top2 r = sm.tops[0];
                for (int w = 1; w < kTokWaves; w++) r = merge(r, sm.tops[w]);
                const float margin = r.v1 - r.v2;
                StepState* st = a->st;
                st->token = r.i1;
                if (a->gen_tok) {
                    const int c = st->gen_count;
                    if (c < a->max_seq) {
                        a->gen_tok[c] = r.i1;
                        a->gen_margin[c] = margin;
                    }
                    st->gen_count = c + 1;
                }
                st->pos = pos + 1;
                st->margin_bits = __float_as_int(margin);
            }
        }
    }
    if (tid == 0) a->epoch[b] = ep;
}

template <int TB, int HD>
hipError_t launch_tok_t(const TokArgs& a, int with_head, hipStream_t st, int grid) {
    hipLaunchKernelGGL((tok_kernel<TB, HD>), dim3(grid), dim3(kTokThreads), 0, st, a, with_head);
    return hipGetLastError();
}

template <int TB, int HD>
int tok_occupancy() {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, tok_kernel<TB, HD>, kTokThreads, 0) != hipSuccess) return 0;
    return n;
}

}  // namespace

bool tok_supported(int n_pts, int hidden, int ffn, int n_heads, int n_kv, int hd) {
    if (n_pts != 127 && n_pts != 217) return false;
    if (hd != 64 && hd != 128) return false;
    if (hidden > kTokMaxCols || ffn > kTokMaxCols || n_heads * hd > kTokMaxCols) return false;
    if (n_kv <= 0 || n_heads % n_kv) return false;
    int occ = 0;
    if (n_pts == 127) occ = hd == 64 ? tok_occupancy<127, 64>() : tok_occupancy<127, 128>();
    else occ = hd == 64 ? tok_occupancy<217, 64>() : tok_occupancy<217, 128>();
    return occ >= 1;
}

int tok_grid() {
    const int n = device_cu_count();
    return n > 0 ? n : 0;
}

hipError_t launch_token(const TokArgs& a, int with_head, hipStream_t st) {
    const int grid = tok_grid();
    if (grid <= 0) return hipErrorInvalidDevice;
    if (a.n_pts == 127)
        return a.hd == 64 ? launch_tok_t<127, 64>(a, with_head, st, grid) : launch_tok_t<127, 128>(a, with_head, st, grid);
    if (a.n_pts == 217)
        return a.hd == 64 ? launch_tok_t<217, 64>(a, with_head, st, grid) : launch_tok_t<217, 128>(a, with_head, st, grid);
    return hipErrorInvalidValue;
}

}  // namespace gsd
