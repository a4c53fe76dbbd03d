// gsd_ffn.hip -- the feed-forward block of one decode token in one launch:
// RMSNorm, gate/up, SwiGLU, down (split over the FFN rows), the rank-2 and
// kink terms and the residual add (gsd_lq_cpu_runtime.py:380-404 with the
// matvec of gsd_lq_cpu_engine.c:129-183).
//
// Block b < nb owns FFN rows 64 b .. 64 b + 63.  Its waves stream the four
// 16-row units of gate and of up (each wave its own 128-column chunks of x,
// the eight row groups of a chunk back to back), form h for the 64 rows, and
// stream column slab b of down: W_down[:, 64 b .. 64 b + 63] h, 32 rows per
// step, the step's partial sums going out as tagged words at once.  The code
// loads run two steps ahead across the gate/up -> down boundary, so the down
// stream starts while the block forms h.  Block s < nslices then reduces
// rows 16 s .. 16 s + 15 over the nb blocks' words.
//
// Arithmetic per 16-row x 16-pair product, as the batch-1 matvec of
// gsd_kernels.hip: v_mfma_f32_16x16x32_f16 with A = the input's (u, v) =
// (xa, xa / 2 + xb sqrt(3) / 2) per pair as fp16 high and low parts after a
// power-of-two prescale (rows 0 / 1; about 2^-22 relative), B = the rows'
// integer codeword fields (r0, r1) from the lane's own copy of the codebook
// in LDS; the fp16 block scale is applied per 64-weight block.
#include "gsd_device.h"
#include "gsd_internal.h"

namespace gsd {
namespace {

constexpr int kFfnWaves = 16;
#ifndef GSD_FFN_DEPTH
#define GSD_FFN_DEPTH 4
#endif
// code steps in flight per wave (a divisor of 8: the row groups of a chunk)
constexpr int kFfnDepth = GSD_FFN_DEPTH;
static_assert(8 % kFfnDepth == 0, "ring depth");
// polling rounds of a reducing block (s_sleep plus a round trip each, ~1 us;
// about 65 ms in all) before its wait counts as timed out; a normal wait is
// a few rounds
constexpr int kFfnSpinLimit = 1 << 16;
constexpr float kS32f = 0.866025403784438646763723170752936183f;   // sqrt(3) / 2

// one tile step: the lane's 16 codes in two halves (h = 0: codes 0-7, 1:
// codes 8-15), each half a 16-row x 32-pair product over two MFMAs (t = 0,
// 1) with the A fragments A0 (half 0) and A1 (half 1); returns the two
// halves' dot products (rows 0 + 1 of D: high + low parts of the input)
template <bool B7>
__device__ __forceinline__ void tile_dots(uint4 cw, const uint32_t* stab, uint32_t lane_off, uint32_t sh7,
                                          const u32x4v (&A0)[2], const u32x4v (&A1)[2], float& r0, float& r1) {
    uint32_t w4[4] = {cw.x, cw.y, cw.z, cw.w};
    if (B7) align7(w4, sh7);
    const unsigned char* tb = reinterpret_cast<const unsigned char*>(stab);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        float4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 2; t++) {
            u32x4v bw;
#pragma unroll
            for (int e = 0; e < 4; e++)
                bw[e] = *reinterpret_cast<const uint32_t*>(tb + code_addr(w4, 4 * (2 * h + t) + e, lane_off, B7));
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, h ? A1[t] : A0[t]),
                                                      __builtin_bit_cast(half8v, bw), d, 0, 0, 0);
        }
        (h ? r1 : r0) = d[0] + d[1];
    }
}

// fp16 high | low parts of (u, v) * sc as the two A-operand dwords of a pair
__device__ __forceinline__ void hilo(float u, float v, float sc, uint32_t& hi, uint32_t& lo) {
    const float uu = u * sc, vv = v * sc;
    const _Float16 uh = (_Float16)uu, vh = (_Float16)vv;
    const _Float16 ul = (_Float16)(uu - (float)uh), vl = (_Float16)(vv - (float)vh);
    hi = (uint32_t)__builtin_bit_cast(uint16_t, uh) | ((uint32_t)__builtin_bit_cast(uint16_t, vh) << 16);
    lo = (uint32_t)__builtin_bit_cast(uint16_t, ul) | ((uint32_t)__builtin_bit_cast(uint16_t, vl) << 16);
}

// dword of pair q (0 .. 63) of a 128-column chunk in the A-operand order the
// MFMA lanes read: ((h * 2 + t) * 4 + lg) * 8 + e for q = 32 h + 8 lg + 4 t
// + e (high part; + 4: low part)
__device__ __forceinline__ int pair_dword(int q) {
    return ((((q >> 5) & 1) * 2 + ((q >> 2) & 1)) * 4 + ((q >> 3) & 3)) * 8 + (q & 3);
}

// P1: 128-column chunks of x per wave (waves at or past the chunk count have
// none); B7: 7-bit code tiles (codebooks of <= 128 points); R2: every tensor
// carries a rank-2 term; OF: the o projection and its residual add first
// (x = x + W_o attn, formed 16 rows per block and handed over as tagged
// words), so a layer's o and FFN are one launch
template <int P1, bool B7, bool R2, bool OF>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4))) ffn_kernel(const FfnArgs a) {
    // arguments used outside the main loops are read where they are used,
    // through the argument segment (the asm keeps the compiler from holding
    // them all in scalar registers across the loops, where they spilled)
    using KA = const __attribute__((address_space(4))) FfnArgs;
    KA* ka = (KA*)__builtin_amdgcn_kernarg_segment_ptr();
    __asm__ volatile("" : "+s"(ka));
    constexpr int NW = kFfnWaves, TBY = B7 ? kTile7 : kTileU8, D = kFfnDepth;
    __shared__ __attribute__((aligned(16))) uint32_t stab[kTableSlots * 64];   // lane copies of the codebook
    __shared__ __attribute__((aligned(16))) uint32_t xop[NW][P1 * 128];       // each wave's x operands
    __shared__ __attribute__((aligned(16))) uint32_t hop[64];                 // the block's h operands
    __shared__ float red[NW][8][16];
    __shared__ float rsum[NW][16];         // slice sums of each wave
    __shared__ float ssq[NW];
    __shared__ float vtp[NW][4];
    __shared__ float ovtp[NW][2];          // OF: each wave's attn . Vt_o[j]
    __shared__ float sS[8];                // R2: S[j] of gate at j, up at 2 + j; OF: S_o[j] at 6 + j
    __shared__ uint32_t hu[3][64];         // R2, lane l: U of gate / up row 64 b + l, down Vt column 64 b + l
    __shared__ float hsc;                  // descale of the h operands
    __shared__ float tk[2];                // down's rank values S[j] * (Vt[j] . h)
    __shared__ uint32_t pres[2][16];       // the slice's rows: residual x (bits), down's U row

    using KU32 = const __attribute__((address_space(4))) uint32_t;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.x;
    // this launch's tag: the block's launch count + 1 (every block's count
    // is the same; the block's own word, read by no other block)
    const unsigned tag = *(KU32*)(a.ctr + b) + 1u;
    if (tid == 0) a.ctr[b] = tag;
    const int lim = a.spin_limit;
    const int hidden = a.hidden, ffn = a.ffn, nb = a.nb, hpad = a.hpad;
    const bool reduces = b < a.nslices;
    const int srow = 16 * b + (lane & 15);   // the slice row of lanes l, l + 16, ...

    // slice inputs (wave 0; lanes 0-15 use them): residual row and down's U
    // row (loaded by every lane of the wave, clamped: no divergent loads)
    uint32_t xres = 0u, dur = 0u;
    if (reduces && wid == 0) {
        const int r = min(srow, hidden - 1);
        xres = __float_as_uint(ka->x[r]);
        if constexpr (R2) dur = reinterpret_cast<const uint32_t*>(ka->dU)[r];
    }

    // OF: block s < nslices first forms rows 16 s .. 16 s + 15 of x + W_o attn
    // (the o projection of the token, gsd_lq_cpu_runtime.py:376-378), the
    // rows every block's gate / up input needs, and publishes them as tagged
    // words (xw)
    const bool work = b < nb, doO = OF && reduces;
    unsigned long long* xw = a.words + (size_t)nb * hpad + 2 * nb + ffn;
    if (work || doO) {
        const int nc = a.nc;
        const int p1 = work && wid < nc ? P1 : 0;   // chunks of this wave: wid + NW p, p < p1
        const int po = doO && wid < nc ? P1 : 0;    // (o: as many input chunks as gate / up)
        const int n1 = 8 * p1;
        const int n2 = work && wid < a.ns2 ? (a.ns2 - 1 - wid) / NW + 1 : 0;
        const int nsteps = n1 + n2;
        const uint32_t lto = tile_lane_off(B7, lane), lso = (uint32_t)(lane & 15);
        const int nrb = a.nrb;

        // ---- prologue.  OF: the wave's chunks of attn and of o's rank-2
        // rows, o's code steps of the block's unit, o's epilogue inputs.
        // Otherwise: x, the norm weights and the rank-2 rows of the wave's
        // chunks.  Then the FFN's epilogue inputs and first code steps.
        float2 av[P1];
        uint32_t avt[P1][2];
        uint4 ocw[P1];
        uint32_t osw[P1];
        uint32_t oug = 0u;
        float osv = 0.f;
        if constexpr (OF) {
            if (po) {
#pragma unroll
                for (int p = 0; p < P1; p++) {
                    const int c0 = (wid + NW * p) * 128 + 2 * lane;
                    av[p] = *reinterpret_cast<const float2*>(ka->attn + c0);
                    if constexpr (R2) {
                        avt[p][0] = *reinterpret_cast<const uint32_t*>(ka->oVt + c0);
                        avt[p][1] = *reinterpret_cast<const uint32_t*>(ka->oVt + hidden + c0);
                    }
                }
#pragma unroll
                for (int p = 0; p < P1; p++) {
                    const size_t t = (size_t)b * nc + wid + NW * p;
                    ocw[p] = tile_load(ka->ocodes + t * TBY + lto);
                    osw[p] = ka->oscales[t * 16 + lso];
                }
            }
            if (R2 && doO && wid == 0) {
                oug = reinterpret_cast<const uint32_t*>(ka->oU)[min(srow, hidden - 1)];
                osv = ka->oS[lane & 1];
            }
        }
        float2 xv[P1], wv[P1];
        uint32_t vt[P1][4];
        auto load_x_aux = [&]() {   // the norm weights and rank-2 rows of the wave's chunks
#pragma unroll
            for (int p = 0; p < P1; p++) {
                const int c0 = (wid + NW * p) * 128 + 2 * lane;
                wv[p] = *reinterpret_cast<const float2*>(ka->norm_w + c0);
                if constexpr (R2) {
                    vt[p][0] = *reinterpret_cast<const uint32_t*>(ka->gVt + c0);
                    vt[p][1] = *reinterpret_cast<const uint32_t*>(ka->gVt + hidden + c0);
                    vt[p][2] = *reinterpret_cast<const uint32_t*>(ka->uVt + c0);
                    vt[p][3] = *reinterpret_cast<const uint32_t*>(ka->uVt + hidden + c0);
                }
            }
        };
        if (!OF && p1) {
#pragma unroll
            for (int p = 0; p < P1; p++)
                xv[p] = *reinterpret_cast<const float2*>(ka->x + (wid + NW * p) * 128 + 2 * lane);
            load_x_aux();
        }
        // wave 0: U rows of the block's gate and up rows, down's Vt columns
        // of the block's slab (lane l: FFN row / column 64 b + l), and the S
        // values of gate (lanes 0-1) and up (lanes 2-3), which read at h time
        // would each put a memory round trip there
        const int frow = 64 * b + lane, fr = min(frow, ffn - 1);
        uint32_t gur = 0u, uur = 0u, dv0 = 0u, dv1 = 0u;
        float gus = 0.f;
        if (R2 && work && wid == 0) {
            gur = reinterpret_cast<const uint32_t*>(ka->gU)[fr];
            uur = reinterpret_cast<const uint32_t*>(ka->uU)[fr];
            dv0 = ka->dVt[fr];
            dv1 = ka->dVt[ffn + fr];
            gus = (lane & 2 ? a.uS : a.gS)[lane & 1];
        }

        auto step_ptr = [&](int s, const unsigned char*& cp, const uint32_t*& sp) {
            s = min(s, nsteps - 1);
            if (s < n1) {
                const int p = s >> 3, rg = s & 7;
                const size_t t = (size_t)min(4 * b + (rg & 3), nrb - 1) * nc + wid + NW * p;
                cp = (rg < 4 ? a.gcodes : a.ucodes) + t * TBY;
                sp = (rg < 4 ? a.gscales : a.uscales) + t * 16;
            } else {
                const size_t t = (size_t)b * a.ns2 + wid + NW * (s - n1);
                cp = a.dcodes + t * TBY;
                sp = a.dscales + t * 16;
            }
        };
        uint4 cw[D];
        uint32_t sw[D];
        int ls = 0;
        // (no loads past the wave's last step: the slice reduction's polls
        // would return behind them)
        auto issue = [&](int i) {
            if (ls >= nsteps) return;
            const unsigned char* cp;
            const uint32_t* sp;
            step_ptr(ls++, cp, sp);
            cw[i] = tile_load(cp + lto);
            sw[i] = sp[lso];
        };
        // (OF: the FFN's first code steps go out once the new x is in: a
        // load returns after every load the wave issued before it, so steps
        // issued earlier would hold back each poll of the new x)
        if (!OF && nsteps > 0) {
#pragma unroll
            for (int i = 0; i < D; i++) issue(i);
        }

        // codebook: entry e of lane l at byte e * 256 + l * 4; wave w
        // writes entries 16 w .. 16 w + 15 (one 64-byte scalar read)
        if (wid * 16 < ka->n_pts) {
            KU32* fp = (KU32*)ka->fields + wid * 16;
            uint32_t fv[16];
#pragma unroll
            for (int j = 0; j < 16; j++) fv[j] = fp[j];
#pragma unroll
            for (int j = 0; j < 16; j++) stab[(wid * 16 + j) * 64 + lane] = fv[j];
        }

        // OF: attn operands as the x operands below (no norm weights), with
        // the wave's o rank-2 partials attn . Vt_o[j]
        float odk0 = 0.f, odk1 = 0.f, dno = 0.f;
        if constexpr (OF) {
            float omx = 0.f;
            if (po) {
#pragma unroll
                for (int p = 0; p < P1; p++) {
                    const float xa = av[p].x, xb = av[p].y;
                    if constexpr (R2) {
                        odk0 = fmaf(xa, h2f((uint16_t)(avt[p][0] & 0xFFFFu)), odk0);
                        odk0 = fmaf(xb, h2f((uint16_t)(avt[p][0] >> 16)), odk0);
                        odk1 = fmaf(xa, h2f((uint16_t)(avt[p][1] & 0xFFFFu)), odk1);
                        odk1 = fmaf(xb, h2f((uint16_t)(avt[p][1] >> 16)), odk1);
                    }
                    const float u = xa, v = fmaf(kS32f, xb, 0.5f * xa);
                    omx = fmaxf(omx, fmaxf(fabsf(u), fabsf(v)));
                    xop[wid][p * 128 + pair_dword(lane)] = __float_as_uint(u);
                    xop[wid][p * 128 + pair_dword(lane) + 4] = __float_as_uint(v);
                }
            }
            omx = wave_max_nonneg(omx);
            if constexpr (R2) {
                odk0 = wave_sum_valu(odk0);
                odk1 = wave_sum_valu(odk1);
            }
            int ex = 0;
            if (omx > 0.f && omx < INFINITY) (void)frexpf(omx, &ex);
            const float up0 = ldexpf(1.f, 14 - ex);
            dno = ldexpf(1.f, ex - 14);
            if (po) {
#pragma unroll
                for (int p = 0; p < P1; p++) {
                    const int o = p * 128 + pair_dword(lane);
                    uint32_t hi, lo;
                    hilo(__uint_as_float(xop[wid][o]), __uint_as_float(xop[wid][o + 4]), up0, hi, lo);
                    xop[wid][o] = hi;
                    xop[wid][o + 4] = lo;
                }
            }
            if (lane == 0) {
                ovtp[wid][0] = odk0;
                ovtp[wid][1] = odk1;
            }
            if (R2 && doO && wid == 0) {
                hu[2][lane] = oug;   // (lanes 0-15: U_o of the slice rows)
                if (lane < 2) sS[6 + lane] = osv;
            }
        }

        // x operands: pair `lane` of chunk p -> (u, v) of x' = x * w (the
        // RMSNorm factor goes on the finished sums), sum of x^2, the rank-2
        // partials x' . Vt[j] over the wave's columns
        float dn1 = 1.f;
        auto stage_x = [&]() {
            float ss = 0.f, mx = 0.f, dk[4] = {0.f, 0.f, 0.f, 0.f};
            if (p1) {
#pragma unroll
                for (int p = 0; p < P1; p++) {
                    ss = fmaf(xv[p].x, xv[p].x, ss);
                    ss = fmaf(xv[p].y, xv[p].y, ss);
                    const float xa = xv[p].x * wv[p].x, xb = xv[p].y * wv[p].y;
                    if constexpr (R2) {
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            dk[r] = fmaf(xa, h2f((uint16_t)(vt[p][r] & 0xFFFFu)), dk[r]);
                            dk[r] = fmaf(xb, h2f((uint16_t)(vt[p][r] >> 16)), dk[r]);
                        }
                    }
                    const float u = xa, v = fmaf(kS32f, xb, 0.5f * xa);
                    mx = fmaxf(mx, fmaxf(fabsf(u), fabsf(v)));
                    xop[wid][p * 128 + pair_dword(lane)] = __float_as_uint(u);
                    xop[wid][p * 128 + pair_dword(lane) + 4] = __float_as_uint(v);
                }
            }
            ss = wave_sum_valu(ss);
            mx = wave_max_nonneg(mx);
            if constexpr (R2) {
#pragma unroll
                for (int r = 0; r < 4; r++) dk[r] = wave_sum_valu(dk[r]);
            }
            if (lane == 0) {
                ssq[wid] = ss;
                vtp[wid][0] = dk[0];
                vtp[wid][1] = dk[1];
                vtp[wid][2] = dk[2];
                vtp[wid][3] = dk[3];
            }
            // power-of-two scale putting the wave's largest |u|, |v| in [2^13, 2^14)
            int ex = 0;
            if (mx > 0.f && mx < INFINITY) (void)frexpf(mx, &ex);
            const float up1 = ldexpf(1.f, 14 - ex);
            dn1 = ldexpf(1.f, ex - 14);
            if (p1) {
#pragma unroll
                for (int p = 0; p < P1; p++) {
                    const int o = p * 128 + pair_dword(lane);
                    uint32_t hi, lo;
                    hilo(__uint_as_float(xop[wid][o]), __uint_as_float(xop[wid][o + 4]), up1, hi, lo);
                    xop[wid][o] = hi;
                    xop[wid][o + 4] = lo;
                }
            }
        };
        if (!OF) stage_x();
        // (every loaded register is stored before the loops: a register
        // whose load is still pending at a use after them would make the
        // compiler drain the code loads in flight there)
        if (R2 && work && wid == 0) {
            hu[0][lane] = gur;
            hu[1][lane] = uur;
            if (!OF) hu[2][lane] = frow < ffn ? (dv0 | (dv1 << 16)) : 0u;
            if (lane < 4) sS[lane] = gus;
        }
        if (!OF && reduces && wid == 0 && lane < 16) {
            pres[0][lane] = xres;
            pres[1][lane] = dur;
        }
        // the argument line of the kink tables (first read at the h step,
        // where a scalar-cache miss would wait behind the streaming loads)
        // into the scalar cache while the launch waits here anyway
        {
            const uint32_t* t = ka->g_rp;
            __asm__ volatile("" ::"s"(t));
        }
        // the codebook and every wave's own operands in LDS
        lds_barrier();

        const uint32_t lane_off = (uint32_t)lane * 4u;
        const uint32_t sh7 = (uint32_t)(lane & 1) * 16u;
        const int m = lane & 15, lg = lane >> 4;
        const uint4* Xw = reinterpret_cast<const uint4*>(xop[wid]);

        if constexpr (OF) {
            // ---- o: the block's 16 rows over the wave's chunks of attn
            if (doO) {
                float acc = 0.f;
                for (int p = 0; p < po; p++) {
                    u32x4v A[2][2];
#pragma unroll
                    for (int h = 0; h < 2; h++)
#pragma unroll
                        for (int t = 0; t < 2; t++) {
                            const uint4 v = Xw[(((p * 2 + h) * 2 + t) * 4 + lg) * 2 + (m & 1)];
                            A[h][t][0] = v.x; A[h][t][1] = v.y; A[h][t][2] = v.z; A[h][t][3] = v.w;
                        }
                    float r0, r1;
                    tile_dots<B7>(ocw[p], stab, lane_off, sh7, A[0], A[1], r0, r1);
                    acc = fmaf(r0, h2f((uint16_t)(osw[p] & 0xFFFFu)), acc);
                    acc = fmaf(r1, h2f((uint16_t)(osw[p] >> 16)), acc);
                }
                if (lane < 16) red[wid][0][lane] = acc * dno;
                lds_barrier();
                if (wid == 0) {
                    // x + (W_o attn + kinks + U_o S_o (Vt_o attn)), gsd_lq_cpu_engine.c:129-183
                    float y = 0.f, d0 = 0.f, d1 = 0.f;
                    for (int w = 0; w < NW; w++) {
                        y += red[w][0][lane & 15];
                        d0 += ovtp[w][0];
                        d1 += ovtp[w][1];
                    }
                    if (ka->o_rp && srow < hidden) {
                        const uint32_t e = ka->o_rp[srow + 1];
                        for (uint32_t i = ka->o_rp[srow]; i < e; i++) y += ka->o_kd[i] * ka->attn[ka->o_kc[i]];
                    }
                    if constexpr (R2) {
                        const uint32_t uw = hu[2][lane & 15];
                        y += h2f((uint16_t)(uw & 0xFFFFu)) * (sS[6] * d0);
                        y += h2f((uint16_t)(uw >> 16)) * (sS[7] * d1);
                    }
                    const float xn = __uint_as_float(xres) + y;
                    if (lane < 16) {
                        pres[0][lane] = __float_as_uint(xn);
                        pres[1][lane] = dur;
                        if (srow < hidden)
                            __hip_atomic_store(xw + srow, ((unsigned long long)tag << 32) | __float_as_uint(xn),
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
            if (work) {
                // ---- x = x + W_o attn of every row the wave's chunks cover,
                // from the blocks that formed them (bounded wait); with it
                // the norm weights and rank-2 rows
                if (p1) load_x_aux();
                if (p1) {
                    const __amdgpu_buffer_rsrc_t rx =
                        __builtin_amdgcn_make_buffer_rsrc(xw, (short)0, hidden * 8, 0x00020000);
                    for (int spins = 0;; spins++) {
                        bool done = true;
#pragma unroll
                        for (int p = 0; p < P1; p++) {
                            const auto q = __builtin_amdgcn_raw_buffer_load_b128(
                                rx, ((wid + NW * p) * 128 + 2 * lane) * 8, 0, 16 /* sc1 */);
                            done = done && q[1] == tag && q[3] == tag;
                            xv[p] = make_float2(__uint_as_float(q[0]), __uint_as_float(q[2]));
                        }
                        if (done) break;
                        if (spins >= lim) {
                            if (ka->err) *ka->err = 1u;
                            break;
                        }
                        __builtin_amdgcn_s_sleep(2);
                    }
                }
                if (nsteps > 0) {
#pragma unroll
                    for (int i = 0; i < D; i++) issue(i);
                }
                stage_x();
                if (R2 && wid == 0) hu[2][lane] = frow < ffn ? (dv0 | (dv1 << 16)) : 0u;
                lds_barrier();   // (also: every wave's o operands read before the x operands replace them)
            }
        }
        if (work) {
        const uint32_t lane_off = (uint32_t)lane * 4u;
        const uint32_t sh7 = (uint32_t)(lane & 1) * 16u;
        const int m = lane & 15, lg = lane >> 4;
        const uint4* Xw = reinterpret_cast<const uint4*>(xop[wid]);

        // x[c] of the FFN input (OF: x + W_o attn, from the tagged words)
        auto xin = [&](int c) -> float {
            if constexpr (!OF) return ka->x[c];
            unsigned long long v;
            int spins = 0;
            while ((unsigned)((v = __hip_atomic_load(xw + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) >> 32) != tag &&
                   spins < lim) {
                if (++spins == lim && ka->err) *ka->err = 1u;
                __builtin_amdgcn_s_sleep(2);
            }
            return __uint_as_float((unsigned)v);
        };

        // ---- gate / up: 8 row groups (gate units 0-3, up units 0-3) per chunk
        float acc[8];
#pragma unroll
        for (int r = 0; r < 8; r++) acc[r] = 0.f;
        // (one chunk's operands live at a time: unrolled, the chunks'
        // operands and addresses would all be live and spill at depth 4)
#pragma clang loop unroll(disable)
        for (int p = 0; p < p1; p++) {
            u32x4v A[2][2];
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint4 v = Xw[(((p * 2 + h) * 2 + t) * 4 + lg) * 2 + (m & 1)];
                    A[h][t][0] = v.x; A[h][t][1] = v.y; A[h][t][2] = v.z; A[h][t][3] = v.w;
                }
#pragma unroll
            for (int rg = 0; rg < 8; rg++) {
                const int i = rg % D;
                float r0, r1;
                const float sc0 = h2f((uint16_t)(sw[i] & 0xFFFFu)), sc1 = h2f((uint16_t)(sw[i] >> 16));
                tile_dots<B7>(cw[i], stab, lane_off, sh7, A[0], A[1], r0, r1);
                issue(i);
                acc[rg] = fmaf(r0, sc0, acc[rg]);
                acc[rg] = fmaf(r1, sc1, acc[rg]);
            }
        }
        if (lane < 16) {
#pragma unroll
            for (int r = 0; r < 8; r++) red[wid][r][lane] = acc[r] * dn1;
        }
        lds_barrier();

        // ---- h of the block's 64 rows (wave 0, lane l: FFN row 64 b + l),
        // and h as the down operand
        if (wid == 0) {
            float sx = 0.f;
            for (int w = 0; w < NW; w++) sx += ssq[w];
            const float inv = 1.0f / sqrtf(sx / (float)hidden + ka->eps);
            const int k = lane >> 4, r = lane & 15;
            float g = 0.f, u = 0.f;
            for (int w = 0; w < NW; w++) {
                g += red[w][k][r];
                u += red[w][4 + k][r];
            }
            g *= inv;
            u *= inv;
            if (frow < ffn) {
                if (ka->g_rp) {
                    const uint32_t e = ka->g_rp[frow + 1];
                    for (uint32_t i = ka->g_rp[frow]; i < e; i++) {
                        const int c = ka->g_kc[i];
                        g += ka->g_kd[i] * ((xin(c) * inv) * ka->norm_w[c]);
                    }
                }
                if (ka->u_rp) {
                    const uint32_t e = ka->u_rp[frow + 1];
                    for (uint32_t i = ka->u_rp[frow]; i < e; i++) {
                        const int c = ka->u_kc[i];
                        u += ka->u_kd[i] * ((xin(c) * inv) * ka->norm_w[c]);
                    }
                }
                if constexpr (R2) {
                    float d0 = 0.f, d1 = 0.f, e0 = 0.f, e1 = 0.f;
                    for (int w = 0; w < NW; w++) {
                        d0 += vtp[w][0];
                        d1 += vtp[w][1];
                        e0 += vtp[w][2];
                        e1 += vtp[w][3];
                    }
                    // tmp_k[j] = S[j] * (x' . Vt[j]) (gsd_lq_cpu_engine.c:110-127)
                    const float tg0 = sS[0] * (d0 * inv), tg1 = sS[1] * (d1 * inv);
                    const float tu0 = sS[2] * (e0 * inv), tu1 = sS[3] * (e1 * inv);
                    const uint32_t gw = hu[0][lane], uw = hu[1][lane];
                    g += h2f((uint16_t)(gw & 0xFFFFu)) * tg0;
                    g += h2f((uint16_t)(gw >> 16)) * tg1;
                    u += h2f((uint16_t)(uw & 0xFFFFu)) * tu0;
                    u += h2f((uint16_t)(uw >> 16)) * tu1;
                }
            }
            // SwiGLU (gsd_lq_cpu_engine.c:96-108); rows past ffn are 0
            const float hv = frow < ffn ? (g / (1.0f + expf(-g))) * u : 0.f;
            if (frow < ffn) {
                ka->h[frow] = hv;
                if (ka->d_rp)   // (down's kinks read h of any block)
                    __hip_atomic_store(a.words + (size_t)nb * hpad + 2 * nb + frow,
                                       ((unsigned long long)tag << 32) | __float_as_uint(hv), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
            // down's rank-2 partials over the slab: h . Vt[j] (S applied
            // by the reducer)
            if constexpr (R2) {
                const uint32_t dvt = hu[2][lane];
                const float p0 = wave_sum_valu(hv * h2f((uint16_t)(dvt & 0xFFFFu)));
                const float q0 = wave_sum_valu(hv * h2f((uint16_t)(dvt >> 16)));
                if (lane < 2)
                    __hip_atomic_store(a.words + (size_t)nb * hpad + 2 * b + lane,
                                       ((unsigned long long)tag << 32) | __float_as_uint(lane ? q0 : p0),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            // pairs (h[2q], h[2q + 1]) as (u, v), prescaled like x
            const float hb = __shfl_xor(hv, 1, 64);
            const bool ev = (lane & 1) == 0;
            const float pu = ev ? hv : 0.f, pv = ev ? fmaf(kS32f, hb, 0.5f * hv) : 0.f;
            const float hm = wave_max_nonneg(fmaxf(fabsf(pu), fabsf(pv)));
            int e2 = 0;
            if (hm > 0.f && hm < INFINITY) (void)frexpf(hm, &e2);
            if (ev) {
                uint32_t hi, lo;
                hilo(pu, pv, ldexpf(1.f, 14 - e2), hi, lo);
                const int q = lane >> 1;
                hop[pair_dword(q)] = hi;
                hop[pair_dword(q) + 4] = lo;
            }
            if (lane == 0) hsc = ldexpf(1.f, e2 - 14);
        }
        lds_barrier();

        // ---- down, slab b: step i = rows 32 sd .. 32 sd + 31, sd = wid + NW i
        const uint4* Hw = reinterpret_cast<const uint4*>(hop);
        u32x4v B2[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint4 v = Hw[(t * 4 + lg) * 2 + (m & 1)];
            B2[t][0] = v.x; B2[t][1] = v.y; B2[t][2] = v.z; B2[t][3] = v.w;
        }
        const float dn2 = hsc;
        unsigned long long* wb = a.words + (size_t)b * hpad;
        auto down_step = [&](int i, int slot) {
            float r0, r1;
            const float sc0 = h2f((uint16_t)(sw[slot] & 0xFFFFu)), sc1 = h2f((uint16_t)(sw[slot] >> 16));
            tile_dots<B7>(cw[slot], stab, lane_off, sh7, B2, B2, r0, r1);
            issue(slot);
            const int row = 32 * (wid + NW * i) + lane;
            const float y = (lane < 16 ? r0 * sc0 : r1 * sc1) * dn2;
            if (lane < 32 && row < hidden)
                __hip_atomic_store(wb + row, ((unsigned long long)tag << 32) | __float_as_uint(y), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        };
        // (phase 1 ends on ring slot 0: 8 steps per chunk)
        int i2 = 0;
        for (; i2 + D <= n2; i2 += D) {
#pragma unroll
            for (int k = 0; k < D; k++) down_step(i2 + k, k);
        }
#pragma unroll
        for (int k = 0; k < D - 1; k++)
            if (i2 + k < n2) down_step(i2 + k, k);
        }
    } else if (reduces && wid == 0 && lane < 16) {
        pres[0][lane] = xres;
        pres[1][lane] = dur;
    }

    // ---- rows 16 s .. 16 s + 15 of x: the nb blocks' partials in block
    // order.  Lane l of wave w reads block 4 w + (l >> 4) + 64 i's word of
    // row 16 s + (l & 15) (128 contiguous bytes per 16 lanes); wave 1 reads
    // the rank words.  Word loads bypass the non-coherent caches (sc1); a
    // word without this launch's tag is polled again (bounded).
    if (!reduces) return;
    constexpr int NI = 4;   // nb <= 256
    const int lgp = lane >> 4;
    {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            a.words, (short)0, (nb * hpad + 2 * nb) * 8, 0x00020000);
        int off[NI];
        bool use[NI];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int p = 4 * wid + lgp + 64 * i;
            use[i] = p < nb && srow < hidden;
            off[i] = use[i] ? (p * hpad + srow) * 8 : 0x7FFFFFF0;
        }
        unsigned long long wv[NI];
        for (int spins = 0;; spins++) {
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const auto w2 = __builtin_amdgcn_raw_buffer_load_b64(rs, off[i], 0, 16 /* sc1 */);
                wv[i] = ((unsigned long long)w2[1] << 32) | w2[0];
            }
            bool done = true;
#pragma unroll
            for (int i = 0; i < NI; i++) done = done && (!use[i] || (unsigned)(wv[i] >> 32) == tag);
            if (done) break;
            if (spins >= lim) {
                if (ka->err) *ka->err = 1u;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < NI; i++) v += use[i] ? __uint_as_float((unsigned)wv[i]) : 0.f;
        v = swap_add16(v, v);        // + the lane 16 apart (another block, same row)
        v = swap_add32(v, v, false);  // + the lanes 32 apart
        if (lane < 16) rsum[wid][lane] = v;
        if (R2 && wid == 1) {
            // down's S (issued ahead of the polls, whose round trip it shares)
            const float ds0 = a.dS[0], ds1 = a.dS[1];
            // rank words: lane l, blocks l + 64 i, both j in one 16-byte load
            int ro[NI];
            bool rok[NI];
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const int p = lane + 64 * i;
                rok[i] = p < nb;
                ro[i] = rok[i] ? (nb * hpad + 2 * p) * 8 : 0x7FFFFFF0;
            }
            unsigned long long w0[NI], w1[NI];
            for (int spins = 0;; spins++) {
#pragma unroll
                for (int i = 0; i < NI; i++) {
                    const auto q = __builtin_amdgcn_raw_buffer_load_b128(rs, ro[i], 0, 16 /* sc1 */);
                    w0[i] = ((unsigned long long)q[1] << 32) | q[0];
                    w1[i] = ((unsigned long long)q[3] << 32) | q[2];
                }
                bool done = true;
#pragma unroll
                for (int i = 0; i < NI; i++)
                    done = done && (!rok[i] || ((unsigned)(w0[i] >> 32) == tag && (unsigned)(w1[i] >> 32) == tag));
                if (done) break;
                if (spins >= lim) {
                    if (ka->err) *ka->err = 1u;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            float d0 = 0.f, d1 = 0.f;
#pragma unroll
            for (int i = 0; i < NI; i++) {
                d0 += rok[i] ? __uint_as_float((unsigned)w0[i]) : 0.f;
                d1 += rok[i] ? __uint_as_float((unsigned)w1[i]) : 0.f;
            }
            d0 = wave_sum_valu(d0);
            d1 = wave_sum_valu(d1);
            if (lane == 0) {
                tk[0] = ds0 * d0;
                tk[1] = ds1 * d1;
            }
        }
    }
    lds_barrier();
    if (wid == 0 && lane < 16 && srow < hidden) {
        float y = 0.f;
        for (int w = 0; w < NW; w++) y += rsum[w][lane];
        if (ka->d_rp) {
            // kink terms of down read h of any block (tagged words)
            const unsigned long long* hw = a.words + (size_t)nb * hpad + 2 * nb;
            const uint32_t e = ka->d_rp[srow + 1];
            for (uint32_t i = ka->d_rp[srow]; i < e; i++) {
                const int c = ka->d_kc[i];
                unsigned long long v;
                int spins = 0;
                while ((unsigned)((v = __hip_atomic_load(hw + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) >> 32) !=
                           tag &&
                       spins < lim) {
                    if (++spins == lim && ka->err) *ka->err = 1u;
                    __builtin_amdgcn_s_sleep(2);
                }
                y += ka->d_kd[i] * __uint_as_float((unsigned)v);
            }
        }
        if constexpr (R2) {
            const uint32_t uw = pres[1][lane];
            y += h2f((uint16_t)(uw & 0xFFFFu)) * tk[0];
            y += h2f((uint16_t)(uw >> 16)) * tk[1];
        }
        ka->x[srow] = __uint_as_float(pres[0][lane]) + y;
    }
}

}  // namespace

size_t ffn_words(int hidden, int ffn) {
    const int nb = ffn / 64, hpad = (hidden + 15) / 16 * 16;
    return (size_t)nb * hpad + 2 * (size_t)nb + (size_t)ffn + (size_t)hidden;
}

bool ffn_supported(int hidden, int ffn) {
    if (hidden <= 0 || ffn <= 0 || hidden % 128 || ffn % 64) return false;
    const int nc = hidden / 128;
    if (!(nc <= kFfnWaves || nc == 2 * kFfnWaves || nc == 4 * kFfnWaves)) return false;
    const int grid = std::max(ffn / 64, hidden / 16);
    return grid <= device_cu_count();
}

hipError_t launch_ffn(const FfnArgs& a0, hipStream_t st) {
    if (!ffn_supported(a0.hidden, a0.ffn)) return hipErrorNotSupported;
    if (!a0.gcodes || !a0.ucodes || !a0.dcodes || !a0.fields || !a0.x || !a0.norm_w || !a0.h || !a0.words ||
        !a0.ctr || a0.n_pts < 1 || a0.n_pts > kTableSlots)
        return hipErrorInvalidValue;
    const bool r2 = a0.gU != nullptr, of = a0.ocodes != nullptr;
    if (r2 && (!a0.uU || !a0.dU || !a0.gS || !a0.uS || !a0.dS || !a0.gVt || !a0.uVt || !a0.dVt))
        return hipErrorInvalidValue;
    if (of && (!a0.oscales || !a0.attn || a0.qd != a0.hidden || (r2 && (!a0.oU || !a0.oS || !a0.oVt))))
        return hipErrorInvalidValue;
    FfnArgs a = a0;
    a.nb = a.ffn / 64;
    a.nslices = a.hidden / 16;
    a.hpad = a.nslices * 16;
    a.nc = a.hidden / 128;
    a.nrb = (a.ffn + 15) / 16;
    a.ns2 = (a.hidden + 31) / 32;
    if (a.spin_limit <= 0) a.spin_limit = kFfnSpinLimit;
    const int grid = std::max(a.nb, a.nslices);
    if (grid > kFfnMaxGrid) return hipErrorNotSupported;
    const int p1 = a.nc <= kFfnWaves ? 1 : a.nc / kFfnWaves;
    const bool b7 = a.n_pts <= 128;
#define GSD_FFN(P, B, R, O)                                                   \
    if (p1 == P && b7 == B && r2 == R && of == O)                             \
    hipLaunchKernelGGL((ffn_kernel<P, B, R, O>), dim3(grid), dim3(1024), 0, st, a)
#define GSD_FFN4(P, B) \
    GSD_FFN(P, B, true, true); else GSD_FFN(P, B, true, false); else GSD_FFN(P, B, false, true); else GSD_FFN(P, B, false, false)
    GSD_FFN4(1, true);
    else GSD_FFN4(1, false);
    else GSD_FFN4(2, true);
    else GSD_FFN4(2, false);
    else GSD_FFN4(4, true);
    else GSD_FFN4(4, false);
#undef GSD_FFN4
#undef GSD_FFN
    return hipGetLastError();
}

}  // namespace gsd
