// gsd_kernels.hip -- gfx950 kernels of the GSD-LQ decode engine.
//
// Hot path: hexmv, the fused unpack + dequant matvec of GSD-LQ packed weights
// (reference semantics: gsd_cpu_hex2d_matvec, gsd_lq_cpu_engine.c:129-183).
// Design for CDNA4 (wave64, 160 KB LDS, HBM3E):
//   * each thread owns fixed 32-column "slots" of the input vector and keeps
//     that slice in VGPRs for the whole launch, so x is read once per block,
//     not once per row;
//   * for every row a slot is one 16-byte global load of codes (16 pairs),
//     adjacent lanes read adjacent 16-byte pieces of the same row, so a wave
//     reads 1 KB contiguous per row: 128-bit, fully coalesced;
//   * codes are expanded through the codebook held in LDS (float2 per code),
//     multiplied with the register-resident x slice in fp32, scaled once per
//     16 pairs by the fp16 block scale;
//   * RB rows are in flight per thread (RB independent 16-byte loads and FMA
//     chains), reduced across the block with cross-lane shuffles + LDS;
//   * prologue fusions: RMSNorm of the input (each block, from its register
//     slice); the rank-k projection tmp_k = S * (Vt x) is computed once, by
//     blocks 0..sum(k)-1, and published to the others through flags;
//   * epilogue fusions: kinks and the U tmp_k term, then store / residual add /
//     SwiGLU of paired gate-up rows.
#include <algorithm>
#include <cstdlib>

#include "gsd_internal.h"
#include "gsd_device.h"

namespace gsd {
namespace {


// 16 codes (one 16-byte load) against the 32 matching x values.
__device__ __forceinline__ float dot16(const uint4 c, const float2* __restrict__ T, const float* xv) {
    float p = 0.f;
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int d = 0; d < 4; d++) {
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const float2 t = T[(w[d] >> (8 * b)) & 0xFFu];
            p = fmaf(t.x, xv[8 * d + 2 * b], p);
            p = fmaf(t.y, xv[8 * d + 2 * b + 1], p);
        }
    }
    return p;
}

// Lattice form of dot16: with codeword (r0 + r1/2, r1*s), s = sqrt(3)/2, a pair
// contributes xa*(r0 + r1/2) + xb*r1*s = u*r0 + v*r1 with u = xa and
// v = xa/2 + s*xb precomputed per column pair (uv holds u, v interleaved).
// The table entry is (r0, r1) as two fp16 (exact integers), so each pair is
// one byte-select address (v_lshlrev_b32 SDWA), one 4-byte LDS read and two
// mixed-precision FMAs (v_fma_mix_f32), all arithmetic in fp32.
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot16_lat(const uint4 c, const half2v* __restrict__ T, const float* uv) {
    float p0 = 0.f, p1 = 0.f;   // r0 and r1 terms: two independent FMA chains
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int d = 0; d < 4; d++) {
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const half2v t = T[(w[d] >> (8 * b)) & 0xFFu];
            p0 = fmaf((float)t.x, uv[8 * d + 2 * b], p0);
            p1 = fmaf((float)t.y, uv[8 * d + 2 * b + 1], p1);
        }
    }
    return p0 + p1;
}

// Cross-lane reduction of 8 per-lane partial sums (one per row of a batch)
// with VALU permutes only: two swap-and-add rounds (v_permlane32_swap,
// v_permlane16_swap) halve the values per lane while doubling their span,
// then DPP adds finish each 16-lane row.  On return, lane 16q holds the
// wave totals of rows 2q (u0) and 2q+1 (u1), q = 0..3.
__device__ __forceinline__ void reduce8(const float (&acc)[8], float& u0, float& u1) {
    const float t0 = swap_add32(acc[0], acc[4], false);   // rows 0 | 4
    const float t1 = swap_add32(acc[1], acc[5], false);   // rows 1 | 5
    const float t2 = swap_add32(acc[2], acc[6], false);   // rows 2 | 6
    const float t3 = swap_add32(acc[3], acc[7], false);   // rows 3 | 7
    u0 = row16_sum(swap_add16(t0, t2));                   // rows 0 | 2 | 4 | 6 per 16 lanes
    u1 = row16_sum(swap_add16(t1, t3));                   // rows 1 | 3 | 5 | 7
}

// Rows of batch b.  Unpaired: RB consecutive rows of one segment.  Paired
// (gate/up + SwiGLU): rows 0-3 of the batch are gate rows r0..r0+3, rows 4-7
// the same rows of up.
struct BatchRows {
    int g0, r0;
};

// Rank-k value `lead` of a launch (segments in order, tmp_k == null ones only):
// tmp_k[j] = S[j] * sum_c ((x[c] * inv) * w[c]) * Vt[j][c]
// (gsd_lq_cpu_engine.c:66-82 then :110-127), published as one 64-bit word.
// All loads of a thread (x, norm weights, Vt) are issued before any is used.
template <int SPT>
__device__ void lowrank_publish(const HexArgs& a, int lead, float* scratch) {
    int g = 0, jj = lead;
    for (; g < a.nseg; g++) {
        const int k = a.seg[g].tmp_k ? 0 : a.seg[g].k;
        if (jj < k) break;
        jj -= k > 0 ? k : 0;
    }
    const HexSeg& sg = a.seg[g];
    const int tid = threadIdx.x, NT = blockDim.x, S = a.cols >> 5;
    float ss = 0.f, d = 0.f;
    float4 xv[SPT][8], wv[SPT][8];
    uint4 vv[SPT][4];
#pragma unroll
    for (int j = 0; j < SPT; j++) {
        const int s = min(tid + j * NT, S - 1);
        const float4* xp = reinterpret_cast<const float4*>(a.x + (size_t)s * 32);
        const float4* wp = reinterpret_cast<const float4*>(a.norm_w ? a.norm_w + (size_t)s * 32 : a.x);
        const uint4* vp = reinterpret_cast<const uint4*>(sg.Vt + (size_t)jj * a.cols + (size_t)s * 32);
#pragma unroll
        for (int q = 0; q < 8; q++) xv[j][q] = xp[q];
        if (a.norm_w) {
#pragma unroll
            for (int q = 0; q < 8; q++) wv[j][q] = wp[q];
        }
#pragma unroll
        for (int q = 0; q < 4; q++) vv[j][q] = vp[q];
    }
#pragma unroll
    for (int j = 0; j < SPT; j++) {
        if (tid + j * NT >= S) continue;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            ss = fmaf(xv[j][q].x, xv[j][q].x, ss); ss = fmaf(xv[j][q].y, xv[j][q].y, ss);
            ss = fmaf(xv[j][q].z, xv[j][q].z, ss); ss = fmaf(xv[j][q].w, xv[j][q].w, ss);
        }
    }
    float inv = 1.f;
    if (a.norm_w) {
        ss = block_sum(ss, scratch);
        inv = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
    }
#pragma unroll
    for (int j = 0; j < SPT; j++) {
        if (tid + j * NT >= S) continue;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            float xe[4] = {xv[j][q].x, xv[j][q].y, xv[j][q].z, xv[j][q].w};
            if (a.norm_w) {
                const float we[4] = {wv[j][q].x, wv[j][q].y, wv[j][q].z, wv[j][q].w};
#pragma unroll
                for (int e = 0; e < 4; e++) xe[e] = (xe[e] * inv) * we[e];
            }
            const uint32_t h0 = (&vv[j][q >> 1].x)[2 * (q & 1)], h1 = (&vv[j][q >> 1].x)[2 * (q & 1) + 1];
            d = fmaf(xe[0], h2f((uint16_t)(h0 & 0xFFFFu)), d);
            d = fmaf(xe[1], h2f((uint16_t)(h0 >> 16)), d);
            d = fmaf(xe[2], h2f((uint16_t)(h1 & 0xFFFFu)), d);
            d = fmaf(xe[3], h2f((uint16_t)(h1 >> 16)), d);
        }
    }
    d = block_sum(d, scratch);
    if (tid == 0)
        __hip_atomic_store(&a.pub[lead], (1ull << 32) | __float_as_uint(d * sg.S[jj]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// TM: 0 = generic float2 codeword tables (one per segment), 1 = lattice
// fields, one table shared by all segments, 2 = lattice fields per segment.
template <int SPT, int NWM, bool ST, int TM>
__global__ void __launch_bounds__(NWM * 64) hexmv_kernel(const HexArgs a) {
    constexpr int RB = 8;
    __shared__ float2 tbl[kMaxSeg][kTableSlots];   // TM > 0: half2 entries, 256 per segment
    __shared__ float red[2][NWM][RB];
    __shared__ float fin[RB];
    __shared__ float tkl[kMaxSeg][kMaxRank];
    __shared__ float scratch[16];
    __shared__ float s_inv;

    const int tid = threadIdx.x, NT = blockDim.x, lane = tid & 63, wid = tid >> 6;
    const int NW = NT >> 6;
    const int S = a.cols >> 5;
    const int nsb = a.cols >> 6;
    const size_t rowbytes = (size_t)(a.cols >> 1);
    const bool paired = a.epilogue == kEpiSwiGLU;

    auto rows_of = [&](int b) {
        BatchRows br;
        if (paired) {
            br.g0 = 0;
            br.r0 = b * (RB / 2);
        } else {
            int g = 0;
            while (g + 1 < a.nseg && b >= a.seg[g + 1].batch0) g++;
            br.g0 = g;
            br.r0 = (b - a.seg[g].batch0) * RB;
        }
        return br;
    };

    uint4 cw[SPT][RB];
    uint32_t sv[SPT][RB];
    uint4 uw[2];   // epilogue threads: U row (k <= 16 fp16) of their row, fetched with the batch
    // Issue every load of batch b: RB x SPT 16-byte code loads and the
    // matching scales, rows and slots clamped in range (results of padding
    // rows/slots are discarded later), no branches between the loads.
    auto issue = [&](int b) {
        const BatchRows br = rows_of(b);
#pragma unroll
        for (int j = 0; j < SPT; j++) {
            const int s = min(tid + j * NT, S - 1);
#pragma unroll
            for (int rr = 0; rr < RB; rr++) {
                const int g = paired ? (rr >> 2) : br.g0;
                const int row = min(br.r0 + (paired ? (rr & 3) : rr), a.seg[g].rows - 1);
                cw[j][rr] = *reinterpret_cast<const uint4*>(a.seg[g].codes + (size_t)row * rowbytes + (size_t)s * 16);
                if (!ST) sv[j][rr] = a.seg[g].scales[(size_t)row * nsb + (s >> 1)];
            }
            if (j == 0 && tid < RB) {
                const int g = paired ? (tid >> 2) : br.g0;
                const int kk = a.seg[g].k;
                if (kk > 0) {
                    const int row = min(br.r0 + (paired ? (tid & 3) : tid), a.seg[g].rows - 1);
                    const uint16_t* up = a.seg[g].U + (size_t)row * kk;
                    // U rows are 2*k bytes: fetch as 16-bit loads into the two vectors
                    uint16_t tmp[16];
#pragma unroll
                    for (int q = 0; q < 16; q++) tmp[q] = q < kk ? up[q] : (uint16_t)0;
                    uw[0] = make_uint4(tmp[0] | (uint32_t)tmp[1] << 16, tmp[2] | (uint32_t)tmp[3] << 16,
                                       tmp[4] | (uint32_t)tmp[5] << 16, tmp[6] | (uint32_t)tmp[7] << 16);
                    uw[1] = make_uint4(tmp[8] | (uint32_t)tmp[9] << 16, tmp[10] | (uint32_t)tmp[11] << 16,
                                       tmp[12] | (uint32_t)tmp[13] << 16, tmp[14] | (uint32_t)tmp[15] << 16);
                }
            }
            if (ST) {
#pragma unroll
                for (int grp = 0; grp < 2; grp++) {
                    const int g = paired ? grp : br.g0;
                    const int ngrp = (a.seg[g].rows + 3) >> 2;
                    const int rg = min((br.r0 >> 2) + (paired ? 0 : grp), ngrp - 1);
                    const uint2 w = *reinterpret_cast<const uint2*>(a.seg[g].scales + ((size_t)rg * nsb + (s >> 1)) * 4);
                    sv[j][4 * grp + 0] = w.x & 0xFFFFu;
                    sv[j][4 * grp + 1] = w.x >> 16;
                    sv[j][4 * grp + 2] = w.y & 0xFFFFu;
                    sv[j][4 * grp + 3] = w.y >> 16;
                }
            }
        }
    };

    // blocks 0..nlead-1 compute the rank-k projections and exit; the matvec
    // blocks follow them
    int nlead = 0;
    for (int g = 0; g < a.nseg; g++)
        if (!a.seg[g].tmp_k) nlead += a.seg[g].k > 0 ? a.seg[g].k : 0;
    if ((int)blockIdx.x < nlead) {
        lowrank_publish<SPT>(a, (int)blockIdx.x, scratch);
        return;
    }
    const int nblk = (int)gridDim.x - nlead;
    int b = (int)blockIdx.x - nlead;
    if (b < a.nbatch) issue(b);   // in flight while the prologue runs

    half2v* ltab = reinterpret_cast<half2v*>(&tbl[0][0]);
    if (TM == 0) {
        for (int g = 0; g < a.nseg; g++) {
            const float2* tg = reinterpret_cast<const float2*>(a.seg[g].table);
            for (int i = tid; i < kTableSlots; i += NT) tbl[g][i] = i < a.seg[g].n_pts ? tg[i] : make_float2(0.f, 0.f);
        }
    } else {
        for (int g = 0; g < (TM == 1 ? 1 : a.nseg); g++) {
            const half2v* fg = reinterpret_cast<const half2v*>(a.seg[g].fields);
            for (int i = tid; i < kTableSlots; i += NT) {
                half2v z; z.x = (_Float16)0.f; z.y = (_Float16)0.f;
                ltab[g * kTableSlots + i] = i < a.seg[g].n_pts ? fg[i] : z;
            }
        }
    }

    // input slice: slot s = tid + j*NT covers columns [32s, 32s+32)
    float xr[SPT][32];
#pragma unroll
    for (int j = 0; j < SPT; j++) {
        const int s = tid + j * NT;
        if (s < S) {
            const float4* xp = reinterpret_cast<const float4*>(a.x + (size_t)s * 32);
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float4 v = xp[q];
                xr[j][4 * q] = v.x; xr[j][4 * q + 1] = v.y; xr[j][4 * q + 2] = v.z; xr[j][4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < 32; q++) xr[j][q] = 0.f;
        }
    }

    // fused RMSNorm (gsd_lq_cpu_engine.c:66-82): x' = (x * inv) * w
    float inv = 1.f;
    if (a.norm_w) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < SPT; j++)
#pragma unroll
            for (int q = 0; q < 32; q++) ss = fmaf(xr[j][q], xr[j][q], ss);
        ss = block_sum(ss, scratch);
        inv = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
#pragma unroll
        for (int j = 0; j < SPT; j++) {
            const int s = tid + j * NT;
            if (s < S) {
                const float4* wp = reinterpret_cast<const float4*>(a.norm_w + (size_t)s * 32);
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const float4 w = wp[q];
                    xr[j][4 * q] = (xr[j][4 * q] * inv) * w.x;
                    xr[j][4 * q + 1] = (xr[j][4 * q + 1] * inv) * w.y;
                    xr[j][4 * q + 2] = (xr[j][4 * q + 2] * inv) * w.z;
                    xr[j][4 * q + 3] = (xr[j][4 * q + 3] * inv) * w.w;
                }
            }
        }
    }
    if (tid == 0) s_inv = inv;
    if (TM != 0) {
        // lattice path: (xa, xb) -> (u, v) = (xa, xa/2 + xb*sqrt(3)/2)
        constexpr float kS32 = 0.866025403784438646763723170752936183f;
#pragma unroll
        for (int j = 0; j < SPT; j++)
#pragma unroll
            for (int q = 0; q < 16; q++) xr[j][2 * q + 1] = fmaf(kS32, xr[j][2 * q + 1], 0.5f * xr[j][2 * q]);
    }

    // rank-k values: given (tmp_k, copied here) or published by the
    // projection blocks (fetched by each epilogue lane when it first needs a
    // segment's values; bit g of `have` marks segment g as fetched)
    unsigned have = 0;
    for (int g = 0; g < a.nseg; g++) {
        if (a.seg[g].k > 0 && a.seg[g].tmp_k) {
            if (tid < a.seg[g].k) tkl[g][tid] = a.seg[g].tmp_k[tid];
            have |= 1u << g;
        }
    }
    __syncthreads();

    int buf = 0;
    for (; b < a.nbatch; b += nblk) {
        const BatchRows br = rows_of(b);
        float acc[RB];
#pragma unroll
        for (int rr = 0; rr < RB; rr++) acc[rr] = 0.f;
#pragma unroll
        for (int j = 0; j < SPT; j++) {
            if (tid + j * NT < S) {
#pragma unroll
                for (int rr = 0; rr < RB; rr++) {
                    const int g = paired ? (rr >> 2) : br.g0;
                    float d;
                    if (TM == 0) d = dot16(cw[j][rr], tbl[g], xr[j]);
                    else d = dot16_lat(cw[j][rr], ltab + (TM == 1 ? 0 : g * kTableSlots), xr[j]);
                    acc[rr] = fmaf(d, h2f((uint16_t)sv[j][rr]), acc[rr]);
                }
            }
        }
        const uint4 uw_cur[2] = {uw[0], uw[1]};
        // next batch's loads fly during the reduction and the epilogue
        if (b + nblk < a.nbatch) issue(b + nblk);

        float u0, u1;
        reduce8(acc, u0, u1);
        if ((lane & 15) == 0) {
            red[buf][wid][2 * (lane >> 4)] = u0;
            red[buf][wid][2 * (lane >> 4) + 1] = u1;
        }
        __syncthreads();
        if (tid < RB) {
            const int rr = tid;
            const int g = paired ? (rr >> 2) : br.g0;
            const int row = br.r0 + (paired ? (rr & 3) : rr);
            const HexSeg& sg = a.seg[g];
            float t = 0.f;
            for (int w = 0; w < NW; w++) t += red[buf][w][rr];
            if (row < sg.rows) {
                if (sg.row_ptr) {
                    const uint32_t e = sg.row_ptr[row + 1];
                    for (uint32_t i = sg.row_ptr[row]; i < e; i++) {
                        const int c = sg.kcols[i];
                        const float xc = a.norm_w ? (a.x[c] * s_inv) * a.norm_w[c] : a.x[c];
                        t += sg.kdel[i] * xc;
                    }
                }
                if (sg.k > 0 && !((have >> g) & 1u)) {
                    // this segment's published words (segments without tmp_k
                    // in order); a bounded wait, normally already satisfied:
                    // after 2^20 polls the error word is set
                    int off = 0;
                    for (int g2 = 0; g2 < g; g2++)
                        if (!a.seg[g2].tmp_k && a.seg[g2].k > 0) off += a.seg[g2].k;
                    int spins = 0;
                    for (int jj = 0; jj < sg.k; jj++) {
                        unsigned long long w;
                        while (((w = __hip_atomic_load(&a.pub[off + jj], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) >> 32) == 0 &&
                               spins < (1 << 20)) {
                            if (++spins == (1 << 20)) *a.err = 1u;
                            __builtin_amdgcn_s_sleep(1);
                        }
                        tkl[g][jj] = __uint_as_float((unsigned)w);
                    }
                    have |= 1u << g;
                }
                const uint32_t uu[8] = {uw_cur[0].x, uw_cur[0].y, uw_cur[0].z, uw_cur[0].w,
                                        uw_cur[1].x, uw_cur[1].y, uw_cur[1].z, uw_cur[1].w};
                for (int jj = 0; jj < sg.k; jj++) t += h2f((uint16_t)(uu[jj >> 1] >> (16 * (jj & 1)))) * tkl[g][jj];
                if (a.epilogue == kEpiStore) sg.out[row] = t;
                else if (a.epilogue == kEpiResidual) a.resid[row] = a.resid[row] + t;
            }
            fin[rr] = t;
        }
        if (a.epilogue == kEpiRopeKV) {
            // segments q, k, v; rows 2i, 2i+1 of a head are one rotation pair
            // (interleaved RoPE, gsd_lq_cpu_engine.c:213-256), evaluated without
            // contraction like the reference; k', v stored as fp16 at pos
            __syncthreads();
            if (tid < RB / 2) {
#pragma clang fp contract(off)
                const RopeKV& r = a.rope;
                const int row = br.r0 + 2 * tid;
                const HexSeg& sg = a.seg[br.g0];
                if (row + 1 < sg.rows) {
                    const int pos = r.pos_dev ? *r.pos_dev : r.pos;
                    const float x0 = fin[2 * tid], x1 = fin[2 * tid + 1];
                    const size_t base = ((size_t)r.layer * r.max_seq + (size_t)pos) * (size_t)r.n_kv * r.hd;
                    if (br.g0 == 2) {
                        r.v_cache[base + row] = f2h(x0);
                        r.v_cache[base + row + 1] = f2h(x1);
                    } else {
                        const float2 cs = r.cs[(size_t)pos * (r.hd >> 1) + ((row % r.hd) >> 1)];
                        const float y0 = x0 * cs.x - x1 * cs.y;
                        const float y1 = x0 * cs.y + x1 * cs.x;
                        if (br.g0 == 0) {
                            sg.out[row] = y0;
                            sg.out[row + 1] = y1;
                        } else {
                            r.k_cache[base + row] = f2h(y0);
                            r.k_cache[base + row + 1] = f2h(y1);
                        }
                    }
                }
            }
        }
        if (paired) {
            __syncthreads();
            if (tid < RB / 2) {
                const int row = br.r0 + tid;
                if (row < a.seg[0].rows) {
                    const float gt = fin[tid], up = fin[tid + RB / 2];
                    a.seg[0].out[row] = (gt / (1.0f + expf(-gt))) * up;
                }
            }
        }
        buf ^= 1;
    }
}

template <int SPT, int NWM, bool ST, int TM>
hipError_t launch_hexmv_t(const HexArgs& a, hipStream_t st, int nt) {
    constexpr int RB = 8;
    HexArgs b = a;
    if (b.epilogue == kEpiSwiGLU) {
        b.nbatch = (b.seg[0].rows + RB / 2 - 1) / (RB / 2);
    } else {
        int nb = 0;
        for (int g = 0; g < b.nseg; g++) {
            b.seg[g].batch0 = nb;
            nb += (b.seg[g].rows + RB - 1) / RB;
        }
        b.nbatch = nb;
    }
    if (b.nbatch == 0) return hipSuccess;
    // persistent grid: as many blocks as are resident on the chip at once
    static int per_cu = 0;
    if (per_cu == 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, hexmv_kernel<SPT, NWM, ST, TM>, nt, 0) != hipSuccess || n < 1)
            n = 1;
        per_cu = n;
    }
    // persistent grid (as many blocks as are resident, each looping over
    // batches with the next batch's loads in flight); GSD_HEXMV_PERSIST=0
    // launches one block per batch instead
    static const int persist = getenv("GSD_HEXMV_PERSIST") ? atoi(getenv("GSD_HEXMV_PERSIST")) : 1;
    const int ncu = device_cu_count() > 0 ? device_cu_count() : 256;
    // blocks 0..nlead-1 publish the rank-k values and exit after one short
    // pass; the matvec blocks follow them (dispatched in order, so a matvec
    // block never waits on a publishing block that is not yet resident)
    int nlead = 0;
    for (int g = 0; g < b.nseg; g++)
        if (!b.seg[g].tmp_k && b.seg[g].k > 0) nlead += b.seg[g].k;
    if (nlead > 0 && (!b.pub || !b.err)) return hipErrorInvalidValue;
    int grid = persist ? ncu * per_cu : b.nbatch;
    if (grid > b.nbatch) grid = b.nbatch;
    grid += nlead;
    hipLaunchKernelGGL((hexmv_kernel<SPT, NWM, ST, TM>), dim3(grid), dim3(nt), 0, st, b);
    return hipGetLastError();
}

// ------------------------------------------------------------------------
// rank-k projection twin: one block per j
// ------------------------------------------------------------------------
__global__ void __launch_bounds__(256) lowrank_kernel(const float* x, const uint16_t* Vt, const float* S,
                                                      float* tmp_k, int cols) {
    __shared__ float scratch[16];
    const int j = blockIdx.x;
    float p = 0.f;
    for (int c = threadIdx.x; c < cols; c += blockDim.x) p = fmaf(x[c], h2f(Vt[(size_t)j * cols + c]), p);
    p = block_sum(p, scratch);
    if (threadIdx.x == 0) tmp_k[j] = p * S[j];
}

__global__ void __launch_bounds__(1024) rmsnorm_kernel(const float* x, const float* w, float* out, int dim, float eps) {
    __shared__ float scratch[16];
    float ss = 0.f;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) ss = fmaf(x[i], x[i], ss);
    ss = block_sum(ss, scratch);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = threadIdx.x; i < dim; i += blockDim.x) out[i] = (x[i] * inv) * w[i];
}

__global__ void vec_add_kernel(float* y, const float* a, const float* b, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = a[i] + b[i];
}

__global__ void swiglu_kernel(const float* g, const float* u, float* out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float gv = g[i];
        out[i] = (gv / (1.0f + expf(-gv))) * u[i];
    }
}

// ------------------------------------------------------------------------
// RoPE + KV append (gsd_lq_cpu_engine.c:185-262).  cos/sin come from the
// host (C library), the rotation is evaluated without contraction so the
// fp16 cache bits equal the reference's for equal inputs.
// ------------------------------------------------------------------------
struct CsInline {
    float2 v[128];
};

__global__ void rope_kv_kernel(float* q, const float* k, const float* v, const RopeKV r, const CsInline csi,
                               int use_inline) {
#pragma clang fp contract(off)
    const int half = r.hd >> 1;
    // token blockIdx.y of a batch (one token: 0): its rows and position
    const int tok = blockIdx.y;
    q += (size_t)tok * r.n_heads * r.hd;
    k += (size_t)tok * r.n_kv * r.hd;
    v += (size_t)tok * r.n_kv * r.hd;
    const int pos = (r.pos_dev ? *r.pos_dev : r.pos) + tok;
    const float2* cs = use_inline ? csi.v : r.cs + (size_t)pos * half;
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    const size_t base = ((size_t)r.layer * r.max_seq + (size_t)pos) * (size_t)r.n_kv * r.hd;
    if (gid < r.n_heads * half) {
        const int h = gid / half, i = gid % half;
        const int i0 = h * r.hd + (r.interleaved ? 2 * i : i);
        const int i1 = h * r.hd + (r.interleaved ? 2 * i + 1 : i + half);
        const float c = cs[i].x, s = cs[i].y;
        const float a = q[i0], b = q[i1];
        q[i0] = a * c - b * s;
        q[i1] = a * s + b * c;
    }
    if (gid < r.n_kv * half) {
        const int h = gid / half, i = gid % half;
        const int d0 = r.interleaved ? 2 * i : i;
        const int d1 = r.interleaved ? 2 * i + 1 : i + half;
        const float c = cs[i].x, s = cs[i].y;
        const float a = k[h * r.hd + d0], b = k[h * r.hd + d1];
        r.k_cache[base + (size_t)h * r.hd + d0] = f2h(a * c - b * s);
        r.k_cache[base + (size_t)h * r.hd + d1] = f2h(a * s + b * c);
    }
    if (gid < r.n_kv * r.hd) r.v_cache[base + gid] = f2h(v[gid]);
}

// ------------------------------------------------------------------------
// GQA decode attention, split over the context (flash-decoding).
// grid = (n_kv, max_splits); a block owns one KV head, all G query heads
// that share it (K/V read once per group, not once per query head) and
// `chunk` (<= 256) positions.  LPP = HD/8 lanes hold one position: each lane
// loads 16 bytes (8 fp16 dims) of K or V, so a wave reads 64/LPP whole rows
// per 16-byte load.  Dot products finish with DPP row reductions; every
// reduction stays in VALU (DPP, permlane swaps) except the final cross-wave
// one.  The block of a KV head's last split merges the per-split
// (max, sum, o) partials, handed over as epoch-tagged words.
// ------------------------------------------------------------------------

constexpr int kAttnStage = 8192;   // floats of LDS staging for the merge (32 KB)

// NW waves per block (NT = 64 NW threads): 16 spread a block's arithmetic
// over the CU's four SIMDs (one split: a block per KV head does all the work;
// split contexts: the partial sums and the merge); 4 where 16 would not fit
// the registers (8 query heads per KV head)
template <int HD, int G, int NW>
__global__ void __launch_bounds__(NW * 64) attn_kernel(const AttnArgs a) {
    constexpr int LPP = HD / 8;          // lanes per position
    constexpr int PPW = 64 / LPP;        // positions per wave per step
    constexpr int PPB = NW * PPW;        // positions per block per step
    // steps whose loads are issued together: a whole chunk (256 positions at
    // most) of K and of V for HD <= 128, so one block has its 128 KB in
    // flight at once (a decode block is alone on its CU: it is latency, not
    // bandwidth, that a shallow issue depth runs into)
    constexpr int UNR = 256 / PPB < 16 ? 256 / PPB : 16;
    __shared__ float sc[G][256];
    __shared__ float part[NW][G][HD];
    __shared__ float ml[2][G];
    constexpr int NT = NW * 64;
    __shared__ float lsp[1][256];          // merging block: every split's exp-sum
    __shared__ float stage[kAttnStage];    // merging block: a batch of the splits' outputs

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int sub = lane % LPP, prow = lane / LPP;
    const int kvh = blockIdx.x;
    // the epoch (used at the end).  Device word (a.dep): the epoch of the
    // last launch on the workspace, read by every wave (a vector value: its
    // wait falls at the first use, at the end); this launch's is the next
    // (0 skipped)
    unsigned ep0;
    if (a.dep) {
        const unsigned e = (unsigned)__hip_atomic_load(a.dep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ep0 = e == 0xFFFFFFFFu ? 0u : e;
    } else {
        ep0 = a.epoch ? a.epoch - 1u : (a.counters ? a.counters[kvh] : 0u);
    }
    const int pos = a.pos_dev ? *a.pos_dev : a.pos;
    const int n = pos + 1;
    const int nsplit = (n + a.chunk - 1) / a.chunk;
    const int split = blockIdx.y;
    if (split >= nsplit) return;
    const float* qz = a.q;
    float* outz = a.out;
    const int t0 = split * a.chunk;
    const int t1 = min(n, t0 + a.chunk);
    const int cn = t1 - t0;
    const size_t rowstride = (size_t)a.n_kv * HD;
    const uint16_t* kb = a.k_cache + (size_t)a.layer * a.max_seq * rowstride + (size_t)kvh * HD + sub * 8;
    const uint16_t* vb = a.v_cache + (size_t)a.layer * a.max_seq * rowstride + (size_t)kvh * HD + sub * 8;

    float qv[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float4* qp = reinterpret_cast<const float4*>(qz + (size_t)(kvh * G + g) * HD + sub * 8);
        const float4 q0 = qp[0], q1 = qp[1];
        qv[g][0] = q0.x; qv[g][1] = q0.y; qv[g][2] = q0.z; qv[g][3] = q0.w;
        qv[g][4] = q1.x; qv[g][5] = q1.y; qv[g][6] = q1.z; qv[g][7] = q1.w;
    }

    // phase A: scores s[g][t] = (q_g . K_t) * sm_scale.  Every load is
    // issued, past the chunk's end clamped to its last row (an L2 hit), so the
    // load counts stay fixed; the V rows of the first batch go out right
    // behind the K rows and arrive while the scores are computed.
    const int nsteps = (cn + PPB - 1) / PPB;
    uint4 kw[UNR], vw[UNR];
    auto kload = [&](int s0) {
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int t = min(t0 + (s0 + u) * PPB + wid * PPW + prow, t1 - 1);
            kw[u] = *reinterpret_cast<const uint4*>(kb + (size_t)t * rowstride);
        }
    };
    auto vload = [&](int s0) {
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int t = min(t0 + (s0 + u) * PPB + wid * PPW + prow, t1 - 1);
            vw[u] = *reinterpret_cast<const uint4*>(vb + (size_t)t * rowstride);
        }
    };
    kload(0);
    vload(0);
    // one batch covers the whole chunk (<= 256 positions, the score buffer)
    // when UNR * PPB >= 256: then the loops run once, known at compile time,
    // and the loads' wait counts stay exact
    const int nend = UNR * PPB >= 256 ? 1 : nsteps;
    for (int s0 = 0; s0 < nend; s0 += UNR) {
        if (s0 > 0) kload(s0);
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            if ((s0 + u) * PPB >= cn) break;   // steps past the context (their loads were clamped)
            const int tl = (s0 + u) * PPB + wid * PPW + prow;
            float kf[8];
            unpack8(kw[u], kf);
#pragma unroll
            for (int g = 0; g < G; g++) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++) d = fmaf(qv[g][e], kf[e], d);
                d = lane_group_sum<LPP>(d);
                if (sub == 0 && tl < cn) sc[g][tl] = d * a.sm_scale;
            }
        }
    }
    __syncthreads();
    // phase B: per head max and exp-sum over the chunk (wave w: heads w, w + NW, ...)
    for (int g = wid; g < G; g += NW) {
        float m = -INFINITY;
        for (int i = lane; i < cn; i += 64) m = fmaxf(m, sc[g][i]);
        m = wave_allmax(m);
        float l = 0.f;
        for (int i = lane; i < cn; i += 64) {
            const float e = expf(sc[g][i] - m);
            sc[g][i] = e;
            l += e;
        }
        l = wave_allsum(l);
        if (lane == 0) { ml[0][g] = m; ml[1][g] = l; }
    }
    __syncthreads();
    // phase C: o[g][d] = sum_t p[g][t] V_t[d]
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.f;
    for (int s0 = 0; s0 < nend; s0 += UNR) {
        if (s0 > 0) vload(s0);
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int tl = (s0 + u) * PPB + wid * PPW + prow;
            if (tl < cn) {
                float vf[8];
                unpack8(vw[u], vf);
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float p = sc[g][tl];
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
                }
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = slot_sum<LPP>(acc[g][e]);
    if (prow == 0) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 8; e++) part[wid][g][sub * 8 + e] = acc[g][e];
    }
    __syncthreads();
    const int group_base = kvh * G;
    // the block's output for head g, dim d: its waves' partial sums in a fixed order
    auto psum = [&](int g, int d) {
        float o = (part[0][g][d] + part[1][g][d]) + (part[2][g][d] + part[3][g][d]);
#pragma unroll
        for (int w = 4; w < NW; w += 4)
            o += (part[w][g][d] + part[w + 1][g][d]) + (part[w + 2][g][d] + part[w + 3][g][d]);
        return o;
    };
    if (nsplit == 1) {
        for (int i = tid; i < G * HD; i += NT) {
            const int g = i / HD, d = i % HD;
            outz[(size_t)(group_base + g) * HD + d] = psum(g, d) * (1.0f / ml[1][g]);
        }
        return;
    }
    // partials [kvh][split][g][2+HD] as epoch-tagged words (every block, all
    // G heads); query head g is merged by the block of split nsplit - 1 - g
    // (g mod nsplit when there are fewer splits than heads): no merge launch,
    // no fence, and the merge reads spread over G blocks
    const unsigned ep = ep0 + 1u;
    const unsigned long long tag = (unsigned long long)ep << 32;
    unsigned long long* wsk = a.ws + (size_t)kvh * a.max_splits * G * (2 + HD);
    {
        unsigned long long* wsb = wsk + (size_t)split * G * (2 + HD);
        for (int i = tid; i < G * HD; i += NT) {
            const int g = i / HD, d = i % HD;
            const float o = psum(g, d);
            __hip_atomic_store(wsb + g * (2 + HD) + 2 + d, tag | __float_as_uint(o), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        if (tid < G) {
            __hip_atomic_store(wsb + tid * (2 + HD), tag | __float_as_uint(ml[0][tid]), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(wsb + tid * (2 + HD) + 1, tag | __float_as_uint(ml[1][tid]), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    const int back = nsplit - 1 - split;
    if (back >= G) return;
    // merge: out = sum_s f_s o_s / sum_s f_s l_s, f_s = exp(m_s - max m), in
    // split order.  Word loads bypass the non-coherent caches (sc1) and go out
    // together (out-of-range offsets read 0); a word without this launch's
    // epoch is waited for (bounded), normally never.  Own split from LDS.
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        wsk, (short)0, nsplit * G * (2 + HD) * 8, 0x00020000);
    auto ld = [&](int w) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, w * 8, 0, 16 /* sc1 */);
        return ((unsigned long long)v[1] << 32) | v[0];
    };
    // (wait_skew: a test-only offset that makes the wait run out)
    const unsigned epw = ep + (unsigned)a.wait_skew;
    const int lim = a.spin_limit > 0 ? a.spin_limit : kAttnSpinLimit;
    auto wait_word = [&](int w) {
        unsigned long long v;
        int spins = 0;
        while (((v = __hip_atomic_load(wsk + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) >> 32) != epw &&
               spins < lim) {
            if (++spins == lim && a.err) *a.err = 1u;
            __builtin_amdgcn_s_sleep(1);
        }
        return __uint_as_float((unsigned)v);
    };
    auto value = [&](unsigned long long v, int w) {
        return (v >> 32) == epw ? __uint_as_float((unsigned)v) : wait_word(w);
    };
    constexpr int SB = kAttnStage / HD;       // splits per staging batch
    constexpr int MAXI = kAttnStage / NT;     // staged words per thread
    unsigned long long hcnt = ~0ull;          // a.dep: the heads done before this one
    for (int g = back; g < G; g += nsplit) {
        __syncthreads();   // (LDS reuse across heads)
        // one round trip: the (max, sum) words of every split and the first
        // batch of output words go out together
        unsigned long long v[MAXI];
        auto stage_issue = [&](int s0) {
            const int sn = min(SB, nsplit - s0);
#pragma unroll
            for (int j = 0; j < MAXI; j++) {
                const int i = tid + NT * j, sp = s0 + i / HD, d = i % HD;
                v[j] = ld(i < sn * HD ? (sp * G + g) * (2 + HD) + 2 + d : -1);
            }
        };
        auto stage_put = [&](int s0) {
            const int sn = min(SB, nsplit - s0);
#pragma unroll
            for (int j = 0; j < MAXI; j++) {
                const int i = tid + NT * j, sp = s0 + i / HD, d = i % HD;
                if (i < sn * HD) stage[i] = sp == split ? psum(g, d) : value(v[j], (sp * G + g) * (2 + HD) + 2 + d);
            }
        };
        const int wm = (tid * G + g) * (2 + HD);   // (valid for tid < nsplit)
        const unsigned long long vm = ld(tid < nsplit ? wm : -1), vl = ld(tid < nsplit ? wm + 1 : -1);
        stage_issue(0);
        for (int sp = tid; sp < nsplit; sp += NT) {
            if (sp == split) {
                sc[0][sp] = ml[0][g];
                lsp[0][sp] = ml[1][g];
            } else if (sp == tid) {
                sc[0][sp] = value(vm, wm);
                lsp[0][sp] = value(vl, wm + 1);
            } else {   // (more splits than threads: not launched, kept general)
                const int w = (sp * G + g) * (2 + HD);
                sc[0][sp] = wait_word(w);
                lsp[0][sp] = wait_word(w + 1);
            }
        }
        stage_put(0);
        __syncthreads();
        // (a.dep: every split's words of the head are in, so every block of
        // the head has read the epoch: the head counts itself done)
        if (a.dep && back == 0 && g == 0 && tid == 0)
            hcnt = __hip_atomic_fetch_add(a.dep + 2, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (wid == 0) {
            float M = -INFINITY;
            for (int sp = lane; sp < nsplit; sp += 64) M = fmaxf(M, sc[0][sp]);
            M = wave_allmax(M);
            for (int sp = lane; sp < nsplit; sp += 64) sc[0][sp] = expf(sc[0][sp] - M);
        }
        __syncthreads();
        float L = 0.f, O = 0.f;
        for (int s0 = 0; s0 < nsplit; s0 += SB) {
            if (s0 > 0) {
                stage_issue(s0);
                stage_put(s0);
                __syncthreads();
            }
            const int sn = min(SB, nsplit - s0);
            if (tid < HD)
                for (int k = 0; k < sn; k++) {
                    const float f = sc[0][s0 + k];
                    L = fmaf(lsp[0][s0 + k], f, L);
                    O = fmaf(stage[k * HD + tid], f, O);
                }
            __syncthreads();
        }
        if (tid < HD) outz[(size_t)(group_base + g) * HD + tid] = O / L;
    }
    // the next launch's epoch base (stream order; the counters mode only)
    if (back == 0 && tid == 0 && a.counters && !a.epoch) a.counters[kvh] = ep;
    // a.dep: the last KV head done advances the epoch (every block of the
    // launch has read it by then) and clears the count
    if (a.dep && back == 0 && tid == 0 && hcnt == (unsigned long long)a.n_kv - 1ull) {
        __hip_atomic_store(a.dep + 2, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.dep, (unsigned long long)ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ------------------------------------------------------------------------
// Decode attention for one token, query heads per KV head G <= 4, head dim
// 64 or 128 (the 7B shape: 32 / 8 heads x 128): the matrix-core kernel.
// Every dispatch fetches its code cold, so the instructions a block executes
// once are kept few: the loads are unrolled (one instruction each), the dot
// products are matrix-core steps, and the per-position weighting of V is a
// rolled loop over V staged in LDS.
//
// grid = (n_kv, max_splits), 8 waves; wave w owns positions
// t0 + pw w .. t0 + pw w + pw - 1 of the block's chunk (pw = chunk / 8;
// the chunk a multiple of 64 up to 256).
// Scores with v_mfma_f32_16x16x32_f16, 16 positions x 32 dims per step:
//   A[m][k] = query head m's dims, m < G: the fp16 high part of q * 2^e,
//             a second step the low part (q = hi + lo to 2^-22; e puts the
//             group's largest |q| near 2^13), rows m >= G zero,
//   B[k][n] = K[position n][dims] as stored (fp16, exact),
//   D lane n (n < 16), element m = the score of head m at position n.
// Softmax in the exp2 domain (scores times log2 e), per wave (max, sum);
// weights e[p][g] go through the wave's LDS to the lanes that hold V[p]
// (16 bytes, 8 dims per lane); the waves' (max, sum, o) meet in LDS.
// With more than one split the blocks hand (max, sum, o) per head over as
// epoch-tagged words; the block of the last split (the fewest positions)
// waits for them and merges.  Rows
// past the context are loaded (clamped to the cache) and masked: their
// score is -inf and their V rows are skipped.
// ------------------------------------------------------------------------
constexpr int kAttnDecSplits = 32;   // splits the matrix-core kernel merges (8192 positions at chunk 256)

// RoPE + append fused in front (one token, host position): the new K and V
// rows (fp32, before RoPE), the pairing and the position's (cos, sin)
struct AttnRope {
    const float* k;
    const float* v;
    int interleaved;
    float2 cs[64];   // head dim <= 128
};

// RP: 0 no RoPE; 1 / 2 RoPE + append in front with the interleaved /
// rotate-half pairing (a template parameter: the pairing then costs no
// selects in the rotation code, which every block runs once)
template <int HD, int G, int PW, int RP>
__device__ __forceinline__ void attn_dec_body(const AttnArgs& a, const AttnRope* rp) {
    constexpr bool ROPE = RP > 0, IL = RP == 1;
    constexpr int NW = 8;                 // waves; PW positions each (8, 16 or 32)
    constexpr int NGRP = (PW + 15) / 16;  // groups of 16 positions (matrix-core steps)
    constexpr int NJ = HD / 32;           // matrix-core steps per 16 positions
    constexpr int LPR = HD / 8;           // lanes per V row
    constexpr int RPI = 64 / LPR;         // V rows per load instruction
    constexpr int NV = PW / RPI;          // V loads per wave
    constexpr float kLog2e = 1.44269504088896340736f;
    static_assert(G == 1 || G == 2 || G == 4, "query heads per KV head");
    static_assert(HD == 64 || HD == 128, "head dim");
    static_assert(PW == 8 || PW == 16 || PW == 32, "positions per wave");
    // V staging of wave w (PW rows x HD fp16), reused for its o partials
    // (4 lane rows x G heads x HD floats: 2048 G bytes at HD 128, 1024 G at
    // HD 64 after a row fold, both within 64 HD bytes)
    __shared__ __attribute__((aligned(16))) uint16_t vs[NW][32 * HD];
    __shared__ __attribute__((aligned(16))) float es[NW][32][4];   // e[p][g] of the wave's positions
    __shared__ float wm[NW][4], wl[NW][4];
    // ROPE: each wave's copy of the group's rotated q rows and of the new K
    // (rotated) and V rows as the cache's fp16
    __shared__ __attribute__((aligned(16))) float rq[ROPE ? NW : 1][ROPE ? G * HD : 1];
    __shared__ __attribute__((aligned(16))) uint16_t rkh[ROPE ? NW : 1][ROPE ? HD : 1];
    __shared__ __attribute__((aligned(16))) uint16_t rvh[ROPE ? NW : 1][ROPE ? HD : 1];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kvh = blockIdx.x, split = blockIdx.y;
    const int t0 = split * a.chunk;
    // the position: from the arguments, or read from device memory; a
    // single-split launch loads its rows before it knows it (they are
    // masked after), a split launch first learns whether its split exists
    const bool spec = a.pos_dev == nullptr || a.max_splits == 1;
    int pos = a.pos;
    if (!spec) {
        pos = *a.pos_dev;
        if (t0 > pos) return;   // (uniform: the whole block leaves)
    }
    const size_t rowstride = (size_t)a.n_kv * HD;
    const size_t lbase = (size_t)a.layer * a.max_seq * rowstride + (size_t)kvh * HD;
    const uint16_t* kb = a.k_cache + lbase;
    const uint16_t* vb = a.v_cache + lbase;
    const int rmax = a.max_seq - 1;
    const int pw0 = t0 + wid * PW;   // the wave's first position
    // this launch's epoch, read before any work: the merging block advances
    // the head's counter once it has every split's words, so each block
    // must have read it by then (a block that read it late, after a fast
    // merger's update, would tag its words with the next launch's epoch).
    // Device word (a.dep): the epoch of the last launch on the workspace,
    // loaded by every wave first of all and taken at the block combine
    unsigned dlast = 0;
    if (a.dep) dlast = (unsigned)__hip_atomic_load(a.dep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned ep = a.epoch ? a.epoch : (a.dep || a.max_splits == 1 ? 0u : a.counters[kvh] + 1u);

    // q (A operand source): lane l, head m = l & 15 (m < G), dims
    // 32 j + 8 (l >> 4) .. + 7; issued first, the K and V rows behind it
    const int m = lane & 15, kg = lane >> 4;
    // ROPE: rotation pairs one per lane and step, first of all: lane l takes
    // pair i = l % (HD / 2) (dims 2i, 2i + 1 interleaved, i and i + HD / 2
    // rotate-half) of the new K row, its V dims 2i, 2i + 1 (lanes < HD / 2),
    // the cos / sin of pair i, and pairs l + 64 k of the group's q rows
    // (query head P / (HD / 2) for pair index P)
    constexpr int NPQ = G * HD / 2, KQ = (NPQ + 63) / 64;
    const int ri = lane % (HD / 2), d0 = IL ? 2 * ri : ri, d1 = IL ? 2 * ri + 1 : ri + HD / 2;
    float2 rcs_ = make_float2(1.f, 0.f), rk = make_float2(0.f, 0.f), rv = make_float2(0.f, 0.f);
    float2 rqv[ROPE ? KQ : 1];
    if constexpr (ROPE) {
        rcs_ = rp->cs[ri];
        const float* kn = rp->k + (size_t)kvh * HD;
        rk = make_float2(kn[d0], kn[d1]);
        rv = reinterpret_cast<const float2*>(rp->v + (size_t)kvh * HD)[ri];
#pragma unroll
        for (int k = 0; k < KQ; k++) {
            const int P = min(lane + 64 * k, NPQ - 1);
            const float* qg = a.q + (size_t)(kvh * G + P / (HD / 2)) * HD;
            rqv[k] = make_float2(qg[d0], qg[d1]);
        }
    }
    float4 qa[NJ][2];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        qa[j][0] = qa[j][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (!ROPE && m < G) {
            const float4* qp = reinterpret_cast<const float4*>(a.q + (size_t)(kvh * G + m) * HD + 32 * j + 8 * kg);
            qa[j][0] = qp[0];
            qa[j][1] = qp[1];
        }
    }
    // K (B operand): lane l, position pw0 + 16 grp + (l & 15), same dims
    uint4 kr[NGRP][NJ];
#pragma unroll
    for (int grp = 0; grp < NGRP; grp++) {
        const int t = min(pw0 + 16 * grp + m, rmax);
#pragma unroll
        for (int j = 0; j < NJ; j++)
            kr[grp][j] = *reinterpret_cast<const uint4*>(kb + (size_t)t * rowstride + 32 * j + 8 * kg);
    }
    // V: lane l, position pw0 + RPI u + l / LPR, dims 8 (l % LPR) .. + 7
    const int vrow = lane / LPR, vcol = 8 * (lane % LPR);
    uint4 vr[NV];
#pragma unroll
    for (int u = 0; u < NV; u++) {
        const int t = min(pw0 + RPI * u + vrow, rmax);
        vr[u] = *reinterpret_cast<const uint4*>(vb + (size_t)t * rowstride + vcol);
    }
    if (spec && a.pos_dev) pos = *a.pos_dev;
    const int n = pos + 1;
    const int nsplit = (n + a.chunk - 1) / a.chunk;
    const int t1 = min(n, t0 + a.chunk);   // the block's positions: t0 .. t1 - 1
    const int te = min(t1, pw0 + PW);      // the wave's: pw0 .. te - 1

    // ROPE: the rotated q rows of the group, written back in place from
    // wave 0's copy once every block of the KV head has read q: by the only
    // block, or by the merging block after every split's words have arrived
    auto write_q = [&]() {
        if (ROPE && wid == 0) {
            float* qg = const_cast<float*>(a.q) + (size_t)kvh * G * HD;
            for (int o = lane * 4; o < G * HD; o += 256)
                *reinterpret_cast<float4*>(qg + o) = *reinterpret_cast<const float4*>(&rq[0][o]);
        }
    };
    if constexpr (ROPE) {
        // RoPE (gsd_lq_cpu_engine.c:213-256), one pair per lane, evaluated
        // without contraction like the reference (the bits of
        // rope_kv_kernel's); the rotated q rows and the new fp16 K / V rows
        // go through the wave's LDS to the lanes that hold them in the
        // matrix-core layout (the lanes holding position pos put the new
        // rows in place of the rows they loaded)
#pragma clang fp contract(off)
        auto rot = [&](float2 x) { return make_float2(x.x * rcs_.x - x.y * rcs_.y, x.x * rcs_.y + x.y * rcs_.x); };
#pragma unroll
        for (int k = 0; k < KQ; k++) {
            const int P = lane + 64 * k;
            if (P < NPQ) {
                const float2 y = rot(rqv[k]);
                float* qd = &rq[wid][(P / (HD / 2)) * HD];
                qd[d0] = y.x;
                qd[d1] = y.y;
            }
        }
        if (lane < HD / 2) {
            const float2 y = rot(rk);
            rkh[wid][d0] = f2h(y.x);
            rkh[wid][d1] = f2h(y.y);
            rvh[wid][2 * ri] = f2h(rv.x);
            rvh[wid][2 * ri + 1] = f2h(rv.y);
            // the new rows to the cache: wave 0 of the block whose chunk
            // holds pos
            if (wid == 0 && pos >= t0 && pos < t0 + a.chunk) {
                uint16_t* kc = const_cast<uint16_t*>(a.k_cache) + lbase + (size_t)pos * rowstride;
                uint16_t* vc = const_cast<uint16_t*>(a.v_cache) + lbase + (size_t)pos * rowstride;
                if (IL) {
                    *reinterpret_cast<uint32_t*>(kc + d0) = (uint32_t)f2h(y.x) | ((uint32_t)f2h(y.y) << 16);
                } else {
                    kc[d0] = f2h(y.x);
                    kc[d1] = f2h(y.y);
                }
                *reinterpret_cast<uint32_t*>(vc + 2 * ri) = (uint32_t)f2h(rv.x) | ((uint32_t)f2h(rv.y) << 16);
            }
        }
        if (m < G) {
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const float4* qp = reinterpret_cast<const float4*>(&rq[wid][m * HD + 32 * j + 8 * kg]);
                qa[j][0] = qp[0];
                qa[j][1] = qp[1];
            }
        }
        // (as bit blends: conditional stores of one value into whichever
        // element matches become a run-time index, and the arrays then leave
        // the registers)
        auto blend = [](uint4& d, const uint4 s, bool c) {
            const uint32_t k = c ? 0xFFFFFFFFu : 0u;
            d = make_uint4((s.x & k) | (d.x & ~k), (s.y & k) | (d.y & ~k), (s.z & k) | (d.z & ~k), (s.w & k) | (d.w & ~k));
        };
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const uint4 kn = *reinterpret_cast<const uint4*>(&rkh[wid][32 * j + 8 * kg]);
#pragma unroll
            for (int grp = 0; grp < NGRP; grp++) blend(kr[grp][j], kn, pw0 + 16 * grp + m == pos);
        }
        {
            const uint4 vn = *reinterpret_cast<const uint4*>(&rvh[wid][vcol]);
#pragma unroll
            for (int u = 0; u < NV; u++) blend(vr[u], vn, pw0 + RPI * u + vrow == pos);
        }
    }

    // power-of-two prescale of the group's q: largest |q| into [2^13, 2^14)
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int h = 0; h < 2; h++)
            mx = fmax_nc(mx, fmax_nc(fmax_nc(fabsf(qa[j][h].x), fabsf(qa[j][h].y)), fmax_nc(fabsf(qa[j][h].z), fabsf(qa[j][h].w))));
    mx = wave_max_valu(mx);
    int ex = 0;
    if (mx > 0.f && mx < INFINITY) (void)frexpf(mx, &ex);
    const float up = ldexpf(1.f, 14 - ex);
    const float scl = ldexpf(1.f, ex - 14) * a.sm_scale * kLog2e;
    half8v ahi[NJ], alo[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const float f[8] = {qa[j][0].x, qa[j][0].y, qa[j][0].z, qa[j][0].w,
                            qa[j][1].x, qa[j][1].y, qa[j][1].z, qa[j][1].w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float s = f[e] * up;
            const _Float16 h = (_Float16)s;
            ahi[j][e] = h;
            alo[j][e] = (_Float16)(s - (float)h);
        }
    }

    // scores of the wave's 32 positions: lanes 0-15, element g = head g
    float sv[2][4];
#pragma unroll
    for (int g = 0; g < 4; g++) sv[1][g] = -INFINITY;   // (PW <= 16: one group)
#pragma unroll
    for (int grp = 0; grp < NGRP; grp++) {
        float4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const half8v b = __builtin_bit_cast(half8v, kr[grp][j]);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[j], b, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[j], b, d, 0, 0, 0);
        }
        const bool ok = pw0 + 16 * grp + m < te;
#pragma unroll
        for (int g = 0; g < 4; g++) sv[grp][g] = ok ? d[g] * scl : -INFINITY;
    }
    // the wave's max and exp-sum per head (lanes 0-15 of each DPP row; the
    // other rows compute on values nobody reads)
    float mw[4], lw[4];
#pragma unroll
    for (int g = 0; g < 4; g++) {
        mw[g] = row16_max(fmax_nc(sv[0][g], sv[1][g]));
        const float mu = mw[g] == -INFINITY ? 0.f : mw[g];
        sv[0][g] = __builtin_amdgcn_exp2f(sv[0][g] - mu);
        sv[1][g] = __builtin_amdgcn_exp2f(sv[1][g] - mu);
        lw[g] = row16_sum(sv[0][g] + sv[1][g]);
    }
    if (lane < 16) {
#pragma unroll
        for (int grp = 0; grp < 2; grp++)
            *reinterpret_cast<float4*>(&es[wid][16 * grp + lane][0]) = make_float4(sv[grp][0], sv[grp][1], sv[grp][2], sv[grp][3]);
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            wm[wid][g] = mw[g];
            wl[wid][g] = lw[g];
        }
    }
    // V rows into the wave's LDS (each lane reads back its own words)
    uint4* vw = reinterpret_cast<uint4*>(&vs[wid][0]);
#pragma unroll
    for (int u = 0; u < NV; u++) vw[u * 64 + lane] = vr[u];

    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.f;
    const int nv_live = (max(te - pw0, 0) + RPI - 1) / RPI;   // loads holding a valid row
    for (int u = 0; u < nv_live; u++) {
        const int p = RPI * u + vrow;
        if (pw0 + p < te) {
            float vf[8];
            unpack8(vw[u * 64 + lane], vf);
            const float4 w4 = *reinterpret_cast<const float4*>(&es[wid][p][0]);
            const float wg[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int e = 0; e < 8; e++) acc[g][e] = fmaf(wg[g], vf[e], acc[g][e]);
        }
    }
    // o partials of the wave's lane rows: HD 128: rows l >> 4 (4 rows);
    // HD 64: rows l >> 3 folded pairwise (row_ror 8) into 4
    float* ob = reinterpret_cast<float*>(&vs[wid][0]);
    if constexpr (HD == 64) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 8; e++)
                acc[g][e] += __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(acc[g][e]), 0x128, 0xF, 0xF, true));
    }
    if (HD == 128 || (lane & 15) < 8) {
        const int r = lane >> 4, c = HD == 128 ? (lane & 15) : (lane & 7);
#pragma unroll
        for (int g = 0; g < G; g++) {
            float4* op = reinterpret_cast<float4*>(ob + (r * G + g) * HD + 8 * c);
            op[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
            op[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
        }
    }
    if (a.dep) {   // this launch's epoch: the next (0 skipped)
        ep = (unsigned)__builtin_amdgcn_readfirstlane((int)dlast) + 1u;
        if (ep == 0u) ep = 1u;
    }
    lds_barrier();

    // the block's (max, sum, o) per head: thread (g, d), waves in order
    const int g = tid / HD, d = tid % HD;
    const bool own = tid < G * HD;
    float M = -INFINITY, L = 0.f, O = 0.f;
    if (own) {
        for (int w = 0; w < NW; w++) M = fmax_nc(M, wm[w][g]);
        for (int w = 0; w < NW; w++) {
            const float f = __builtin_amdgcn_exp2f(wm[w][g] - M);   // (-inf: an empty wave, 0)
            const float* o = reinterpret_cast<const float*>(&vs[w][0]);
            const float s = (o[(0 * G + g) * HD + d] + o[(1 * G + g) * HD + d]) + (o[(2 * G + g) * HD + d] + o[(3 * G + g) * HD + d]);
            L = fmaf(f, wl[w][g], L);
            O = fmaf(f, s, O);
        }
    }
    float* outp = a.out + (size_t)(kvh * G + g) * HD + d;
    if (nsplit == 1) {
        if (own) *outp = O / L;
        write_q();
        return;
    }

    // hand-over: words [kvh][split][g][2 + HD]; the block of the last split
    // merges (blocks start in index order, so every other split's block
    // has started before it and finishes without it)
    const unsigned long long tag = (unsigned long long)ep << 32;
    constexpr int WPH = 2 + HD;   // words per head
    unsigned long long* wsk = a.ws + (size_t)kvh * a.max_splits * G * WPH;
    if (own) {
        unsigned long long* wsb = wsk + ((size_t)split * G + g) * WPH;
        __hip_atomic_store(wsb + 2 + d, tag | __float_as_uint(O), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == 0) {
            __hip_atomic_store(wsb, tag | __float_as_uint(M), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(wsb + 1, tag | __float_as_uint(L), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // merge: out = sum_s f_s o_s / sum_s f_s l_s with f_s = 2^(m_s - max m).
    // The G HD outputs of the KV head come in slices of 64 (query head
    // o / HD, dim o % HD); the blocks of the last nm splits merge, block
    // split nsplit - 1 - r taking slices r, r + nm, ...  With one merger
    // (a grid that may not be resident at once) it is the last split's
    // block: blocks start in index order, so every other split's block has
    // started before it and finishes without it; several mergers wait on
    // blocks after their own, so the host allows them only when every block
    // of the grid fits on the device at once.
    constexpr int NSL = G * HD / 64;
    const int nm = min(nsplit, min(max(a.mergers, 1), NSL));
    const int r = nsplit - 1 - split;
    if (r >= nm) return;
    // the tag the merge waits for (wait_skew: a test-only offset that makes
    // the wait run out) and its bound
    const unsigned epw = ep + (unsigned)a.wait_skew;
    const int lim = a.spin_limit > 0 ? a.spin_limit : kAttnSpinLimit;
    unsigned long long hcnt = ~0ull;   // a.dep: the heads done before this one
    // a.dep: the last KV head done advances the epoch (every block of the
    // launch has read it by then) and clears the count
    auto head_done = [&]() {
        if (a.dep && tid == 0 && hcnt == (unsigned long long)a.n_kv - 1ull) {
            __hip_atomic_store(a.dep + 2, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.dep, (unsigned long long)ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(wsk, (short)0, nsplit * G * WPH * 8, 0x00020000);
    if (nsplit <= NW && nm < NSL) {
        // At most 8 splits and fewer mergers than slices: wave w merges slice
        // r + nm w on its own, each lane one output over every split in order
        // (no LDS, no barrier: a block with several slices takes them at
        // once, where the loop below would take them one after another);
        // polled as below.
        const int sl = r + nm * wid;
        if (sl < NSL) {
            const int o = sl * 64 + lane, g2 = o / HD, d2 = o % HD;
            int vo[NW], vml[NW];
#pragma unroll
            for (int s = 0; s < NW; s++) {
                vml[s] = s < nsplit ? (s * G + g2) * WPH * 8 : 0x7FFFFFF0;
                vo[s] = s < nsplit ? vml[s] + (2 + d2) * 8 : 0x7FFFFFF0;
            }
            unsigned long long wo[NW], wmx[NW], wsm[NW];
            for (int spins = 0;; spins++) {
#pragma unroll
                for (int s = 0; s < NW; s++) {
                    auto w2 = __builtin_amdgcn_raw_buffer_load_b64(rs, vo[s], 0, 16 /* sc1 */);
                    wo[s] = ((unsigned long long)w2[1] << 32) | w2[0];
                    w2 = __builtin_amdgcn_raw_buffer_load_b64(rs, vml[s], 0, 16);
                    wmx[s] = ((unsigned long long)w2[1] << 32) | w2[0];
                    w2 = __builtin_amdgcn_raw_buffer_load_b64(rs, vml[s], 8, 16);
                    wsm[s] = ((unsigned long long)w2[1] << 32) | w2[0];
                }
                bool done = true;
#pragma unroll
                for (int s = 0; s < NW; s++)
                    done = done && (s >= nsplit || ((unsigned)(wo[s] >> 32) == epw && (unsigned)(wmx[s] >> 32) == epw &&
                                                    (unsigned)(wsm[s] >> 32) == epw));
                if (done) break;
                if (spins == lim) {   // (bounded, as below)
                    if (a.err) *a.err = 1u;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            // (a.dep: wave 0 of the last split's block has seen every
            // split's words, so every block of the head has read the epoch)
            if (a.dep && r == 0 && tid == 0)
                hcnt = __hip_atomic_fetch_add(a.dep + 2, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            float M2 = -INFINITY;
#pragma unroll
            for (int s = 0; s < NW; s++)
                if (s < nsplit) M2 = fmax_nc(M2, __uint_as_float((unsigned)wmx[s]));
            float L2 = 0.f, O2 = 0.f;
#pragma unroll
            for (int s = 0; s < NW; s++)
                if (s < nsplit) {
                    const float f = __builtin_amdgcn_exp2f(__uint_as_float((unsigned)wmx[s]) - M2);
                    L2 = fmaf(f, __uint_as_float((unsigned)wsm[s]), L2);
                    O2 = fmaf(f, __uint_as_float((unsigned)wo[s]), O2);
                }
            a.out[(size_t)(kvh * G + g2) * HD + d2] = O2 / L2;
        }
        // (wave 0 always has a slice: it has seen every split's words)
        if (r == 0) {
            if (tid == 0 && a.counters && !a.epoch) a.counters[kvh] = ep;   // (counters mode only)
            head_done();
            write_q();
        }
        return;
    }
    // Thread (wave w, lane l): output l of the slice over splits w, w + 8,
    // w + 16, w + 24; its o, max and sum words (the latter two
    // the same address across the wave) loaded together, bypassing the
    // non-coherent caches (sc1), again until every word of a split below
    // nsplit has this launch's epoch (bounded).  Offsets past the words
    // read 0 (buffer bounds).  Then (max, sum, o) of the wave's splits,
    // and the 8 waves' combined by wave 0 through LDS, in a fixed order.
    constexpr int KS = kAttnDecSplits / NW;   // splits per wave
    float* mlo = reinterpret_cast<float*>(&vs[0][0]);   // [3][NW][64]
    lds_barrier();   // (every wave is past its reads of vs above)
    for (int sl = r; sl < NSL; sl += nm) {
        const int o = sl * 64 + lane, g2 = o / HD, d2 = o % HD;
        int vo[KS], vml[KS];
#pragma unroll
        for (int k = 0; k < KS; k++) {
            const int s = wid + NW * k;
            vml[k] = s < nsplit ? (s * G + g2) * WPH * 8 : 0x7FFFFFF0;
            vo[k] = s < nsplit ? vml[k] + (2 + d2) * 8 : 0x7FFFFFF0;
        }
        unsigned long long wo[KS], wmx[KS], wsm[KS];
        for (int spins = 0;; spins++) {
#pragma unroll
            for (int k = 0; k < KS; k++) {
                auto w2 = __builtin_amdgcn_raw_buffer_load_b64(rs, vo[k], 0, 16 /* sc1 */);
                wo[k] = ((unsigned long long)w2[1] << 32) | w2[0];
                w2 = __builtin_amdgcn_raw_buffer_load_b64(rs, vml[k], 0, 16);
                wmx[k] = ((unsigned long long)w2[1] << 32) | w2[0];
                w2 = __builtin_amdgcn_raw_buffer_load_b64(rs, vml[k], 8, 16);
                wsm[k] = ((unsigned long long)w2[1] << 32) | w2[0];
            }
            bool done = true;
#pragma unroll
            for (int k = 0; k < KS; k++)
                done = done && (wid + NW * k >= nsplit ||
                                ((unsigned)(wo[k] >> 32) == epw && (unsigned)(wmx[k] >> 32) == epw &&
                                 (unsigned)(wsm[k] >> 32) == epw));
            if (done) break;
            // (bounded, about 0.2 s: a merger may wait for blocks dispatched
            // after it, which take the CU slots the other blocks free as
            // they finish; kernels of other streams holding the CUs only
            // delay that)
            if (spins == lim) {
                if (a.err) *a.err = 1u;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        float mp = -INFINITY, lp = 0.f, op = 0.f;
#pragma unroll
        for (int k = 0; k < KS; k++)
            if (wid + NW * k < nsplit) mp = fmax_nc(mp, __uint_as_float((unsigned)wmx[k]));
#pragma unroll
        for (int k = 0; k < KS; k++)
            if (wid + NW * k < nsplit) {
                const float f = __builtin_amdgcn_exp2f(__uint_as_float((unsigned)wmx[k]) - mp);
                lp = fmaf(f, __uint_as_float((unsigned)wsm[k]), lp);
                op = fmaf(f, __uint_as_float((unsigned)wo[k]), op);
            }
        mlo[(0 * NW + wid) * 64 + lane] = mp;
        mlo[(1 * NW + wid) * 64 + lane] = lp;
        mlo[(2 * NW + wid) * 64 + lane] = op;
        lds_barrier();
        // (a.dep: every wave has seen its splits' words, so every block of
        // the head has read the epoch)
        if (a.dep && r == 0 && sl == 0 && tid == 0)
            hcnt = __hip_atomic_fetch_add(a.dep + 2, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (wid == 0) {
            float M2 = mlo[lane];
#pragma unroll
            for (int w = 1; w < NW; w++) M2 = fmax_nc(M2, mlo[w * 64 + lane]);
            float L2 = 0.f, O2 = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float f = __builtin_amdgcn_exp2f(mlo[w * 64 + lane] - M2);   // (-inf: no split, 0)
                L2 = fmaf(f, mlo[(NW + w) * 64 + lane], L2);
                O2 = fmaf(f, mlo[(2 * NW + w) * 64 + lane], O2);
            }
            a.out[(size_t)(kvh * G + g2) * HD + d2] = O2 / L2;
        }
        lds_barrier();
    }
    // (the last split's block) every split's block has read the counter
    // and q: the next launch's epoch base (stream order), q written back
    if (r == 0) {
        if (tid == 0 && a.counters && !a.epoch) a.counters[kvh] = ep;   // (counters mode only)
        head_done();
        write_q();
    }
}

template <int HD, int G, int PW>
__global__ void __launch_bounds__(512) attn_dec_kernel(const AttnArgs a) {
    attn_dec_body<HD, G, PW, 0>(a, nullptr);
}
template <int HD, int G, int PW, bool IL>
__global__ void __launch_bounds__(512) attn_rope_kernel(const AttnArgs a, const AttnRope r) {
    attn_dec_body<HD, G, PW, IL ? 1 : 2>(a, &r);
}

// The step state of the next decode launch (token, position); the error word
// is cleared only with reset_err, so a bounded wait that ran out in an
// earlier launch of the same call stays visible to the host.
__global__ void set_step_kernel(StepState* st, int token, int pos, int reset_err) {
    st->token = token;
    st->pos = pos;
    st->gen_count = 0;
    st->margin_bits = 0;
    if (reset_err) st->err = 0u;
}

__global__ void embed_kernel(const uint16_t* embed, const int* token, float* x, int hidden,
                             unsigned long long* clear, int nclear, unsigned* epoch) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < hidden) x[i] = h2f(embed[(size_t)(*token) * hidden + i]);
    if (i < nclear) clear[i] = 0ull;
    if (i == 0 && epoch) *epoch += 1u;   // the token counter of the fused attention tags
}


// the greedy step's outputs: the token and margin (stand-alone call, st
// null), or the step state, the generated token list and the position
__device__ __forceinline__ void argmax_finish(const Top2 r, StepState* st, int* gen_tok, float* gen_margin, int advance,
                                              int c0, int p0) {
    const float margin = r.v1 - r.v2;
    if (!st) {
        gen_tok[0] = r.i1;
        gen_margin[0] = margin;
        return;
    }
    st->token = r.i1;
    if (gen_tok) {
        gen_tok[c0] = r.i1;
        gen_margin[c0] = margin;
        st->gen_count = c0 + 1;
    }
    if (advance) st->pos = p0 + 1;
    st->margin_bits = __float_as_int(margin);
}

__global__ void __launch_bounds__(1024) argmax_kernel(const float* logits, int n, StepState* st, int* gen_tok,
                                                      float* gen_margin, int advance) {
    __shared__ Top2 sw[16];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    // the step state thread 0 updates at the end, read before the logits (a
    // read there would cost one more memory round trip)
    int c0 = 0, p0 = 0;
    if (tid == 0 && st) {
        c0 = st->gen_count;
        p0 = st->pos;
    }
    Top2 t{-INFINITY, -INFINITY, 0x7FFFFFFF};
    // 32 independent coalesced loads per thread per round: one round for a
    // 32768-entry vocabulary
    for (int base = tid; base < n; base += 1024 * 32) {
        float v[32];
#pragma unroll
        for (int u = 0; u < 32; u++) {
            const int i = base + u * 1024;
            v[u] = i < n ? logits[i] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < 32; u++) {
            const int i = base + u * 1024;
            if (i < n) t = merge(t, Top2{clean(v[u]), -INFINITY, i});
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        Top2 u{__shfl_xor(t.v1, o, 64), __shfl_xor(t.v2, o, 64), __shfl_xor(t.i1, o, 64)};
        t = merge(t, u);
    }
    if (lane == 0) sw[wid] = t;
    __syncthreads();
    if (tid == 0) {
        Top2 r = sw[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) r = merge(r, sw[w]);
        argmax_finish(r, st, gen_tok, gen_margin, advance, c0, p0);
    }
}

// The greedy step of the decode graph over kArgBlocks blocks: one block's
// loads of a 32768-entry vocabulary (128 KB through one CU's outstanding
// misses) took ~11 us.  Block b takes entries b * per .. b * per + per - 1,
// keeps (top1, top2, first index of top1) in index order, and hands it over
// as three tagged words (tag: the block's launch count + 1, as every block
// runs each launch); the last block (dispatched last, so every other block
// has started) polls the others' words (bounded: a wait that runs out sets
// st->err), merges them and its own, and finishes as argmax_kernel.  Merging is order-free: the largest value
// with the lowest index is a total order, the runner-up the second largest
// of the union.
__device__ __forceinline__ Top2 top2_add(Top2 t, float c, int i) {
    // i above every index seen: a tie keeps the earlier index
    const bool gt = c > t.v1;
    t.v2 = fmaxf(t.v2, fminf(t.v1, c));
    t.v1 = gt ? c : t.v1;
    t.i1 = gt ? i : t.i1;
    return t;
}
__device__ __forceinline__ Top2 wave_top2(Top2 t) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        Top2 u{__shfl_xor(t.v1, o, 64), __shfl_xor(t.v2, o, 64), __shfl_xor(t.i1, o, 64)};
        t = merge(t, u);
    }
    return t;
}
__global__ void __launch_bounds__(256) argmax_blocks_kernel(const float* logits, int n, StepState* st, int* gen_tok,
                                                            float* gen_margin, int advance, unsigned long long* words,
                                                            unsigned* ctr) {
    __shared__ Top2 sw[4];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int b = blockIdx.x, nb = gridDim.x;
    const bool last = b == nb - 1;
    const unsigned tag = ctr[b] + 1u;   // (the block's own word)
    int c0 = 0, p0 = 0;
    if (last && tid == 0 && st) {
        c0 = st->gen_count;
        p0 = st->pos;
    }
    const int per = (n + nb - 1) / nb, e0 = b * per, e1 = min(n, e0 + per);
    Top2 t{-INFINITY, -INFINITY, 0x7FFFFFFF};
    constexpr int K = 8;
    for (int base = e0 + tid; base < e1; base += 256 * K) {
        float v[K];
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = base + 256 * k;
            v[k] = i < e1 ? logits[i] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = base + 256 * k;
            if (i < e1) t = top2_add(t, clean(v[k]), i);
        }
    }
    t = wave_top2(t);
    if (lane == 0) sw[wid] = t;
    __syncthreads();
    if (!last) {
        if (tid == 0) {
            const Top2 r = merge(merge(sw[0], sw[1]), merge(sw[2], sw[3]));
            unsigned long long* w = words + 3 * (size_t)b;
            const unsigned long long tg = (unsigned long long)tag << 32;
            __hip_atomic_store(w, tg | __float_as_uint(r.v1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(w + 1, tg | __float_as_uint(r.v2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(w + 2, tg | (unsigned)r.i1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ctr[b] = tag;
        }
        return;
    }
    if (wid != 0) return;
    // lane j < nb - 1: block j's words, polled until all carry this tag
    Top2 o{-INFINITY, -INFINITY, 0x7FFFFFFF};
    if (lane < nb - 1) {
        const unsigned long long* w = words + 3 * (size_t)lane;
        unsigned long long a0, a1, a2;
        for (int spins = 0;; spins++) {
            a0 = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            a1 = __hip_atomic_load(w + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            a2 = __hip_atomic_load(w + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((unsigned)(a0 >> 32) == tag && (unsigned)(a1 >> 32) == tag && (unsigned)(a2 >> 32) == tag) break;
            if (spins == (1 << 16)) {   // (bounded, ~65 ms)
                if (st) st->err = 1u;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        o = Top2{__uint_as_float((unsigned)a0), __uint_as_float((unsigned)a1), (int)(unsigned)a2};
    }
    o = wave_top2(o);
    if (lane == 0) {
        const Top2 r = merge(o, merge(merge(sw[0], sw[1]), merge(sw[2], sw[3])));
        ctr[b] = tag;
        argmax_finish(r, st, gen_tok, gen_margin, advance, c0, p0);
    }
}

// Plain 16-byte streaming copy (HBM calibration: its FETCH_SIZE/WRITE_SIZE per
// dispatch against its known size gives the counter scale).
__global__ void __launch_bounds__(256) copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}

__global__ void fill_u32_kernel(unsigned* p, unsigned v, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// enumeration decode: index -> (r0, r1) of the radius-R hexagon
__global__ void unpack_kernel(const uint8_t* codes, int64_t n, int R, int32_t* idx, int8_t* r01) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int c = codes[i];
    idx[i] = c;
    int rem = c, r0 = -R;
    for (; r0 <= R; r0++) {
        const int cnt = 2 * R + 1 - (r0 < 0 ? -r0 : r0);
        if (rem < cnt) break;
        rem -= cnt;
    }
    const int lo = r0 < 0 ? -R - r0 : -R;
    r01[2 * i] = (int8_t)r0;
    r01[2 * i + 1] = (int8_t)(lo + rem);
}

// ------------------------------------------------------------------------
// hexmv4: the fused unpack + dequant matvec on the matrix cores.
//
// Per 64-weight block the reference computes scale * sum_p xy[code_p] . x_p
// (gsd_lq_cpu_engine.c:129-183).  In lattice form a pair contributes
// u*r0 + v*r1 with (u, v) = (xa, xa/2 + xb*sqrt(3)/2) and (r0, r1) the
// codeword's integer fields, which fp16 holds exactly.  One
// v_mfma_f32_16x16x32_f16 then evaluates 16 rows x 16 pairs:
//   B[k][n] = fields of row n (lane n & 15, 4 pairs per lane from the 16-byte
//             code word of the tiled layout, one LDS lookup each),
//   A[m][k] = x side: row m = 0 the fp16 high part of (u, v) * 2^e, row 1 the
//             fp16 low part (x = hi + lo to 2^-22); rows 2..15 repeat them
//             and feed only rows of D that are never read,
//   D[m][n] lands in lane n: element 0 + element 1 = the 16-pair dot product
//             (fp16 x fp16 products are exact, accumulation fp32).
// The per-row fp16 scale is applied after each 32-pair block.  VALU work per
// pair is one v_perm_b32 (LDS address of the lane's own copy of the codebook:
// code << 8 | lane * 4, so the 64 lanes never share a bank).
//
// Work split: one block of W waves per CU takes row-blocks (16 rows) in turn;
// its waves split the 128-column chunks of a row-block (16-byte code loads,
// kMv4Depth chunks in flight per wave) and reduce through LDS; wave 0's lanes 0-15
// run the epilogue.  For the paired gate/up launch the waves form two groups
// (gate row-block, up row-block of the same rows).  A wave only ever reads
// its own chunks of x, so it stages them itself (its own LDS region and
// power-of-two prescale), and the RMSNorm factor multiplies the finished
// sums: nothing waits for all of x before the weights stream.
// ------------------------------------------------------------------------
constexpr int kMv4MaxWaves = 16;
// code steps (1 KB per wave each) in flight per wave.  Measured on the 7B
// layer set: depth 2 streams the gate/up launch as fast as 4 (the CU's 16
// waves keep 32 KB in flight) and, with the main loop unrolled over half as
// many steps, fetches less code per launch (41-42 us per layer set against
// 43.5 at depth 4, 50-53 at depths 6-8, 50 at depth 1)
constexpr int kMv4Depth = 2;
// units per block whose epilogue inputs (residual, RoPE cos/sin, rank-k
// factors) the prologue stages in LDS; the launcher keeps every block within it
constexpr int kMv4PreUnits = 8;

// x'[c] of the launch (RMSNorm applied when norm_w is set), as the reference
// forms it: (x * inv) * w.
__device__ __forceinline__ float xnorm(const HexArgs& a, int c, float inv) {
    return a.norm_w ? (a.x[c] * inv) * a.norm_w[c] : a.x[c];
}

// Rank-k value `lead` of a launch (segments without tmp_k, in order):
// S[j] * sum_c x'[c] * Vt[j][c] (gsd_lq_cpu_engine.c:110-127), published as
// one 64-bit word 1 << 32 | float bits.
__device__ __forceinline__ void mv4_publish(const HexArgs& a, int lead, float* scratch) {
    int g = 0, jj = lead;
    for (; g < a.nseg; g++) {
        const int k = a.seg[g].tmp_k ? 0 : a.seg[g].k;
        if (jj < k) break;
        jj -= k > 0 ? k : 0;
    }
    const HexSeg& sg = a.seg[g];
    float inv = 1.f;
    if (a.norm_w) {
        float ss = 0.f;
        for (int c = threadIdx.x; c < a.cols; c += blockDim.x) ss = fmaf(a.x[c], a.x[c], ss);
        ss = block_sum(ss, scratch);
        inv = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
    }
    float d = 0.f;
    const uint16_t* vt = sg.Vt + (size_t)jj * a.cols;
    for (int c = threadIdx.x; c < a.cols; c += blockDim.x) d = fmaf(xnorm(a, c, inv), h2f(vt[c]), d);
    d = block_sum(d, scratch);
    if (threadIdx.x == 0)
        __hip_atomic_store(&a.pub[lead], (1ull << 32) | __float_as_uint(d * sg.S[jj]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}


// TB > 0: every segment uses the same codebook of TB points, held at a
// static LDS address; TB == 0: per-segment codebooks in dynamic LDS.
// LR: rank-k terms.  0: none (the rank-k machinery is not compiled in: the
// epilogue code is inlined once per pipeline step of the main loop, and a
// smaller kernel runs faster); 1: ranks <= 2, projections computed by every
// block from its own staging of x (kLrSlots); 3: as 1 when every segment
// has rank exactly 2 and no tmp_k (every Precision tensor; fewer
// instructions per launch); 2: any rank, projections published by leading
// blocks.  EPI: the epilogue (HexEpilogue), or -1 to read it from the
// arguments.
// ------------------------------------------------------------------------
// Decode attention of one KV head inside the q/k/v launch, positions
// 0 .. pos with pos < 8 PW (gsd_lq_cpu_engine.c:264-330): the arithmetic of
// attn_dec_body for one split of 8 waves x PW positions (PW 8, 16 or 32: the
// short-context graph's tier of 64, 128 or 256 positions, so that a wave's
// share of the V weighting and of the matrix-core steps follows the
// context), with q and the new
// K / V rows taken from the words the q/k/v epilogue publishes (that launch
// is still writing them), and the cache rows of the earlier positions
// loaded at the start, while the matvec blocks run.  The part after the wait
// runs twice: first on a zero q with no output, while the words are still
// outstanding, which brings its code into the instruction cache (every
// launch starts with a cold one, and the fetch of straight-line code is what
// the short tail after the wait would otherwise spend), then on the words.
// ------------------------------------------------------------------------
// Inputs of the attention blocks, by value (the kernel's argument block is
// read through scalar loads in the matvec path)
struct FaIn {
    const uint16_t* k_cache;
    const uint16_t* v_cache;
    const int* pos_dev;
    const unsigned long long* words;
    float* out;
    unsigned* err;
    int layer, max_seq, n_kv, n_heads;
    float sm_scale;
};

// 16-byte load through a global pointer
__device__ __forceinline__ uint4 gload4(const __attribute__((address_space(1))) uint16_t* p) {
    const u32x4v v = *reinterpret_cast<const __attribute__((address_space(1))) u32x4v*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

template <int HD, int G, int PW>
__device__ __forceinline__ void attn_fa_block(const FaIn a, int kvh, unsigned tag) {
    constexpr int NW = 8, NGRP = (PW + 15) / 16, NJ = HD / 32, LPR = HD / 8, RPI = 64 / LPR, NV = PW / RPI;
    static_assert(PW == 8 || PW == 16 || PW == 32, "positions per wave");
    constexpr int NQ = G * HD, NT = NQ + HD;   // words taken: q rows, then K and V pairs
    constexpr float kLog2e = 1.44269504088896340736f;
    static_assert(G == 1 || G == 2 || G == 4, "query heads per KV head");
    static_assert(HD == 64 || HD == 128, "head dim");
    __shared__ __attribute__((aligned(16))) uint16_t vs[NW][32 * HD];   // V staging, then o partials
    __shared__ __attribute__((aligned(16))) float es[NW][32][4];        // e[p][g] of the wave's positions
    __shared__ float wm[NW][4], wl[NW][4];
    __shared__ __attribute__((aligned(16))) float qs[NQ];               // q rows of the group
    __shared__ __attribute__((aligned(16))) uint32_t kvn[HD];           // new K row, then V row (fp16 pairs)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (wid >= NW) return;
    using KI32 = const __attribute__((address_space(4))) int;
    const int pos = *(KI32*)a.pos_dev;
    const size_t rowstride = (size_t)a.n_kv * HD;
    const size_t lbase = (size_t)a.layer * a.max_seq * rowstride + (size_t)kvh * HD;
    const uint16_t* kb = a.k_cache + lbase;
    const uint16_t* vb = a.v_cache + lbase;
    const int rmax = a.max_seq - 1;
    const int pw0 = wid * PW;   // the wave's first position
    const int m = lane & 15, kg = lane >> 4;
    const int vrow = lane / LPR, vcol = 8 * (lane % LPR);
    for (int i = tid; i < NQ; i += NW * 64) qs[i] = 0.f;
    const int n = pos + 1;
    const int te = min(n, pw0 + PW);   // the wave's positions: pw0 .. te - 1
    const int g = tid / HD, d = tid % HD;
    const bool own = tid < G * HD;
    const int qd = a.n_heads * HD, kvd = a.n_kv * HD;
    const unsigned long long* wq = a.words + (size_t)kvh * NQ;
    const unsigned long long* wk = a.words + qd + (size_t)kvh * (HD / 2);
    const unsigned long long* wv = wk + kvd / 2;
    int nit = 2;
    __asm__ volatile("" : "+s"(nit));   // a loop, not two copies of its body
#pragma clang loop unroll(disable)
    for (int it = 0; it < nit; it++) {
        lds_barrier();   // q zeroed (first pass) / the previous pass's LDS reads done
        // K (B operand): lane l, position pw0 + 16 grp + (l & 15), dims
        // 32 j + 8 (l >> 4) .. + 7; V: lane l, position pw0 + RPI u + l / LPR,
        // dims 8 (l % LPR) .. + 7 (the second pass finds them in L2, and
        // loads them ahead of its wait)
        // (the bases pass through an asm at each pass: hoisted out of the
        // loop, the 16 row addresses would stay live, and spill, across it)
        using GU16 = const __attribute__((address_space(1))) uint16_t;
        GU16* kbi = (GU16*)kb;
        GU16* vbi = (GU16*)vb;
        int rm = rmax;
        __asm__ volatile("" : "+s"(kbi), "+s"(vbi), "+s"(rm));
        uint4 kr[NGRP][NJ];
#pragma unroll
        for (int grp = 0; grp < NGRP; grp++) {
            const int t = min(pw0 + 16 * grp + m, rm);
#pragma unroll
            for (int j = 0; j < NJ; j++)
                kr[grp][j] = gload4(kbi + (size_t)t * rowstride + 32 * j + 8 * kg);
        }
        uint4 vr[NV];
#pragma unroll
        for (int u = 0; u < NV; u++) {
            const int t = min(pw0 + RPI * u + vrow, rm);
            vr[u] = gload4(vbi + (size_t)t * rowstride + vcol);
        }
        // V rows into the wave's LDS (each lane reads back its own words)
        uint4* vw = reinterpret_cast<uint4*>(&vs[wid][0]);
#pragma unroll
        for (int u = 0; u < NV; u++) vw[u * 64 + lane] = vr[u];
        if (it == 1) {
            // the words of this KV head, all with this launch's tag: each
            // wave waits for its own share (no block barrier per round), then
            // the block meets once (bounded)
            for (int spins = 0;; spins++) {
                unsigned stale = 0u;
                for (int i = tid; i < NT; i += NW * 64) {
                    const unsigned long long* p = i < NQ ? wq + i : (i < NQ + HD / 2 ? wk + (i - NQ) : wv + (i - NQ - HD / 2));
                    const unsigned long long w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if ((unsigned)(w >> 32) != tag) stale = 1u;
                    else if (i < NQ) qs[i] = __uint_as_float((unsigned)w);
                    else kvn[i - NQ] = (unsigned)w;
                }
                if (__ballot(stale != 0u) == 0ull) break;
                if (spins == (1 << 18)) {
                    if (a.err) *a.err = 1u;
                    break;
                }
            }
            lds_barrier();
        }
        // position pos takes the new K and V rows (the words; in the first
        // pass whatever the LDS holds), selected where the rows are used
        uint4 knew[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++) knew[j] = *reinterpret_cast<const uint4*>(&kvn[16 * j + 4 * kg]);
        const uint4 vnew = *reinterpret_cast<const uint4*>(&kvn[HD / 2 + vcol / 2]);

        // q of the group's heads (A operand: lane l, head m = l & 15 < G)
        float4 qa[NJ][2];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            qa[j][0] = qa[j][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < G) {
                const float4* qp = reinterpret_cast<const float4*>(&qs[m * HD + 32 * j + 8 * kg]);
                qa[j][0] = qp[0];
                qa[j][1] = qp[1];
            }
        }
        // power-of-two prescale of q: largest |q| into [2^13, 2^14); fp16 high + low parts
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int h = 0; h < 2; h++)
                mx = fmax_nc(mx, fmax_nc(fmax_nc(fabsf(qa[j][h].x), fabsf(qa[j][h].y)), fmax_nc(fabsf(qa[j][h].z), fabsf(qa[j][h].w))));
        mx = wave_max_valu(mx);
        int ex = 0;
        if (mx > 0.f && mx < INFINITY) (void)frexpf(mx, &ex);
        const float up = ldexpf(1.f, 14 - ex);
        const float scl = ldexpf(1.f, ex - 14) * a.sm_scale * kLog2e;
        half8v ahi[NJ], alo[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const float f[8] = {qa[j][0].x, qa[j][0].y, qa[j][0].z, qa[j][0].w,
                                qa[j][1].x, qa[j][1].y, qa[j][1].z, qa[j][1].w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float s = f[e] * up;
                const _Float16 h = (_Float16)s;
                ahi[j][e] = h;
                alo[j][e] = (_Float16)(s - (float)h);
            }
        }
        // scores of the wave's positions: lanes 0-15, element g = head g
        // (PW <= 16: one group, the second all -inf)
        float sv[2][4];
#pragma unroll
        for (int gg = 0; gg < 4; gg++) sv[1][gg] = -INFINITY;
#pragma unroll
        for (int grp = 0; grp < NGRP; grp++) {
            float4v dd = {0.f, 0.f, 0.f, 0.f};
            const bool at = pw0 + 16 * grp + m == pos;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const half8v b = __builtin_bit_cast(half8v, at ? knew[j] : kr[grp][j]);
                dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[j], b, dd, 0, 0, 0);
                dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[j], b, dd, 0, 0, 0);
            }
            const bool ok = pw0 + 16 * grp + m < te;
#pragma unroll
            for (int gg = 0; gg < 4; gg++) sv[grp][gg] = ok ? dd[gg] * scl : -INFINITY;
        }
        // the wave's max and exp2-sum per head
        float mw[4], lw[4];
#pragma unroll
        for (int gg = 0; gg < 4; gg++) {
            mw[gg] = row16_max(fmax_nc(sv[0][gg], sv[1][gg]));
            const float mu = mw[gg] == -INFINITY ? 0.f : mw[gg];
            sv[0][gg] = __builtin_amdgcn_exp2f(sv[0][gg] - mu);
            sv[1][gg] = __builtin_amdgcn_exp2f(sv[1][gg] - mu);
            lw[gg] = row16_sum(sv[0][gg] + sv[1][gg]);
        }
        if (lane < 16) {
#pragma unroll
            for (int grp = 0; grp < NGRP; grp++)
                *reinterpret_cast<float4*>(&es[wid][16 * grp + lane][0]) = make_float4(sv[grp][0], sv[grp][1], sv[grp][2], sv[grp][3]);
        }
        if (lane == 0) {
#pragma unroll
            for (int gg = 0; gg < 4; gg++) {
                wm[wid][gg] = mw[gg];
                wl[wid][gg] = lw[gg];
            }
        }
        if (pos >= pw0 && pos < pw0 + PW && vrow == (pos - pw0) % RPI)   // the lanes that staged row pos
            vw[((pos - pw0) / RPI) * 64 + lane] = vnew;
        float acc[G][8];
#pragma unroll
        for (int gg = 0; gg < G; gg++)
#pragma unroll
            for (int e = 0; e < 8; e++) acc[gg][e] = 0.f;
        const int nv_live = (max(te - pw0, 0) + RPI - 1) / RPI;   // loads holding a valid row
        for (int u = 0; u < nv_live; u++) {
            const int p = RPI * u + vrow;
            if (pw0 + p < te) {
                float vf[8];
                unpack8(vw[u * 64 + lane], vf);
                const float4 w4 = *reinterpret_cast<const float4*>(&es[wid][p][0]);
                const float wg[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                for (int gg = 0; gg < G; gg++)
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[gg][e] = fmaf(wg[gg], vf[e], acc[gg][e]);
            }
        }
        // o partials of the wave's lane rows (HD 64: rows folded pairwise)
        float* ob = reinterpret_cast<float*>(&vs[wid][0]);
        if constexpr (HD == 64) {
#pragma unroll
            for (int gg = 0; gg < G; gg++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    acc[gg][e] += __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(acc[gg][e]), 0x128, 0xF, 0xF, true));
        }
        if (HD == 128 || (lane & 15) < 8) {
            const int rr = lane >> 4, c = HD == 128 ? (lane & 15) : (lane & 7);
#pragma unroll
            for (int gg = 0; gg < G; gg++) {
                float4* op = reinterpret_cast<float4*>(ob + (rr * G + gg) * HD + 8 * c);
                op[0] = make_float4(acc[gg][0], acc[gg][1], acc[gg][2], acc[gg][3]);
                op[1] = make_float4(acc[gg][4], acc[gg][5], acc[gg][6], acc[gg][7]);
            }
        }
        lds_barrier();
        // the block's (max, sum, o) per head: thread (g, d), waves in order
        if (own) {
            float M = -INFINITY, L = 0.f, O = 0.f;
            for (int w = 0; w < NW; w++) M = fmax_nc(M, wm[w][g]);
            for (int w = 0; w < NW; w++) {
                const float f = __builtin_amdgcn_exp2f(wm[w][g] - M);   // (-inf: an empty wave, 0)
                const float* o = reinterpret_cast<const float*>(&vs[w][0]);
                const float s = (o[(0 * G + g) * HD + d] + o[(1 * G + g) * HD + d]) + (o[(2 * G + g) * HD + d] + o[(3 * G + g) * HD + d]);
                L = fmaf(f, wl[w][g], L);
                O = fmaf(f, s, O);
            }
            if (it == 1) a.out[(size_t)(kvh * G + g) * HD + d] = O / L;
        }
    }
}

// FAHD > 0: the q/k/v launch with the decode attention of positions < 8 FAPW
// in its last a.fa.nkv blocks (one per KV head, head dim FAHD, FAG query heads
// per KV head); the matvec blocks are the others and run a.mv.nw waves each
// (the attention runs 8), and the RoPE + K/V epilogue also publishes q and
// the new K/V rows as tagged words (HexArgs::FusedAttn).
template <int TB, int LR, int EPI, int FAHD = 0, int FAG = 0, int DEP = kMv4Depth, int FAPW = 32>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4))) hexmv4_kernel(const HexArgs a) {
    constexpr bool FA = FAHD > 0;
    if constexpr (FA) {
        const int nmv = (int)gridDim.x - a.fa.nkv;
        if ((int)blockIdx.x >= nmv) {
            using KU32c = const __attribute__((address_space(4))) uint32_t;
            const unsigned tag = *(KU32c*)a.fa.epoch_dev * 64u + (unsigned)a.rope.layer + 1u;
            const FaIn fi{a.rope.k_cache, a.rope.v_cache, a.rope.pos_dev, a.fa.words, a.fa.out, a.err,
                          a.rope.layer, a.rope.max_seq, a.rope.n_kv, a.rope.n_heads, a.fa.sm_scale};
            attn_fa_block<FAHD, FAG, FAPW>(fi, (int)blockIdx.x - nmv, tag);
            return;
        }
        if ((int)(threadIdx.x >> 6) >= a.mv.nw) return;
    }
    // (whole 16-entry slices: every filling wave writes 16 entries, the
    // padding ones from the zero padding of the field table)
    __shared__ __attribute__((aligned(16))) uint32_t stab[TB > 0 ? ((TB + 15) & ~15) * 64 : 1];
    __shared__ float red[2][kMv4MaxWaves][16];
    __shared__ float tkl[kMaxSeg][kMaxRank];
    // LR 1 and 3 form the projections in the block; LR 3: every segment has
    // rank exactly 2 and no tmp_k (each Precision tensor), so the slot masks
    // and the rank-1 and tmp_k paths are not compiled in
    constexpr bool kIn = LR == 1 || LR == 3, kR2 = LR == 3;
    // RMSNorm of x: always in the fused q/k/v (RoPE) and gate/up (SwiGLU)
    // launches, never in the residual ones (the launcher sends any other
    // combination to the generic kernel), read from the arguments otherwise
    constexpr int kNorm = EPI == kEpiResidual ? 0 : (EPI == kEpiSwiGLU || EPI == kEpiRopeKV ? 1 : -1);
    // LR 1 / 3: each wave's partial rank-k dot products over its own columns
    // (times S[j]), slot r = j (paired launch: the wave's group's segment) or
    // 2 g + j, wave index last
    constexpr int kVS = !kIn ? 1 : (EPI == kEpiResidual || EPI == kEpiSwiGLU ? 2 : 2 * kMaxSeg);
    static_assert(!kIn || kVS == 2 || kVS == 2 * kMaxSeg, "rank-k slot counts");
    __shared__ float vtp[kVS][kIn ? kMv4MaxWaves : 1];
    __shared__ float scratch[32];
    __shared__ float ssq[kMv4MaxWaves];   // sum of x^2 over each wave's columns
    // epilogue inputs of the block's units (written and read by the epilogue
    // lanes, wave 0 lanes 0-15)
    __shared__ float lpre[EPI == kEpiResidual || EPI < 0 ? kMv4PreUnits : 1][16];
    __shared__ float2 lcs[EPI == kEpiRopeKV || EPI < 0 ? kMv4PreUnits : 1][16];
    __shared__ uint32_t lup[LR > 0 ? kMv4PreUnits : 1][2][16];
    __shared__ float lsk[2 * kMaxSeg];   // LR 1 / 3: S[j] of segment g at 2 g + j
    extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];

    // wid in a scalar register: the segment selections below (seg_of) then
    // read the kernel arguments with scalar loads; a per-lane index makes
    // them vector loads whose vmcnt wait drains the code loads in flight
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    // segment g of the arguments, indexed in the kernel-argument segment (a
    // select chain over a.seg[0..2] becomes an indexed private copy of the
    // whole argument block)
    using KSeg = const __attribute__((address_space(4))) HexSeg;
    using KArgs = const __attribute__((address_space(4))) HexArgs;
    KArgs* kargs = (KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    __asm__ volatile("" : "+s"(kargs));
    KSeg* kseg = kargs->seg;
    {
        // one round trip, before any other read of the arguments, brings
        // every 64-byte line of them into the scalar cache; the reads below,
        // which depend on each other, then hit instead of missing one after
        // another
        using KW = const __attribute__((address_space(4))) uint32_t;
        KW* kw = reinterpret_cast<KW*>(kargs);
        static_assert(sizeof(HexArgs) <= 10 * 64, "argument lines touched below");
        uint32_t t0 = kw[0], t1 = kw[16], t2 = kw[32], t3 = kw[48], t4 = kw[64];
        uint32_t t5 = kw[80], t6 = kw[96], t7 = kw[112], t8 = kw[128];
        uint32_t t9 = kw[(sizeof(HexArgs) - 4) / 4];
        __asm__ volatile("" ::"s"(t0), "s"(t1), "s"(t2), "s"(t3), "s"(t4), "s"(t5), "s"(t6), "s"(t7), "s"(t8), "s"(t9)
                         : "memory");
    }
    // (argument values used right away pass through an asm placed after the
    // batch, so nothing waits for them before the batch is out)
    unsigned bdim = blockDim.x;
    if constexpr (FA) bdim = (unsigned)a.mv.nw * 64u;
    int cols0 = a.cols, epi0 = a.epilogue;
    int P = a.mv.P, wrl = a.mv.wr_log2, nunits = a.mv.nunits, ub1 = a.mv.ub1, ub2 = a.mv.ub2;
    int units_q = a.mv.units_q, units_r = a.mv.units_r, su = a.mv.su, su_u0 = a.mv.su_u0;
    __asm__ volatile("" : "+s"(bdim), "+s"(cols0), "+s"(epi0), "+s"(P), "+s"(wrl), "+s"(nunits), "+s"(ub1), "+s"(ub2),
                     "+s"(units_q), "+s"(units_r), "+s"(su), "+s"(su_u0));
    const int epi = EPI >= 0 ? EPI : epi0;
    const int NW = (int)(bdim >> 6);
    const int nc = (cols0 + 127) >> 7;
    const bool paired = epi == kEpiSwiGLU;
    // waves of a row-block group: a power of two dividing the chunk count
    const int G = paired ? 2 : 1, WR = 1 << wrl, grp = wid >> wrl, wr = wid & (WR - 1);
    using KU32 = const __attribute__((address_space(4))) uint32_t;

    // rank-k publishing blocks first
    int nlead = 0;
    if constexpr (LR == 2)
        for (int g = 0; g < a.nseg; g++)
            if (!a.seg[g].tmp_k && a.seg[g].k > 0) nlead += a.seg[g].k;
    if (LR == 2 && (int)blockIdx.x < nlead) {
        mv4_publish(a, (int)blockIdx.x, scratch);
        return;
    }
    const int nblk = (int)gridDim.x - nlead - (FA ? a.fa.nkv : 0);

    // units: paired -> row-block rb of gate and up; else the row-blocks of
    // the segments in order (first units ub1, ub2 of segments 1, 2)
    auto seg_of = [&](int u) {   // segment of a unit for this wave
        if (paired) return grp;
        return u >= ub2 ? 2 : (u >= ub1 ? 1 : 0);
    };
    auto ubase = [&](int g) { return g == 0 ? 0 : (g == 1 ? ub1 : ub2); };
    const int toff1 = TB == 0 ? a.seg[0].n_pts * 256 : 0;
    const int toff2 = TB == 0 && a.nseg > 1 ? toff1 + a.seg[1].n_pts * 256 : toff1;
    const int tab_bytes = TB == 0 && a.nseg > 2 ? toff2 + a.seg[2].n_pts * 256 : toff2;
    auto toff = [&](int g) { return g == 0 ? 0 : (g == 1 ? toff1 : toff2); };

    // this wave's steps: P chunks (wr, wr + WR, ...) of each of the block's
    // units in turn (units u0, u0 + nblk, ...); P is the same for every wave
    // (WR divides nc), so unit ends, and their barriers, fall on the same step
    // in all waves.  The load cursor runs DEP steps ahead of the compute
    // cursor; both advance by compare-and-reset, and per-unit base pointers
    // are recomputed only when a unit starts.  Past the block's last unit
    // the load cursor stays on that unit (valid addresses, unused data,
    // lines the block has just read: a shared unit there would have every
    // block's surplus loads meet on the same few HBM channels).
    // P >= 1 chunks per wave and unit (WR divides nc)
    const int u0 = (int)blockIdx.x - nlead;
    const int my_full = u0 < nunits ? units_q + (u0 < units_r ? 1 : 0) : 0;
    // half units (paired launches with a shared codebook and no rank-k term;
    // with the rank-2 term the extra cursor state spilled scalar registers
    // and the launch ran ~3 us slower in decode):
    // the block's last unit is then rows 8 hs .. 8 hs + 7 of gate and of up
    // of unit su_unit, in the 16 columns of the matrix-core tile (lanes
    // 0-7: gate, 8-15: up), and each wave takes P / 2 of its chunks (group
    // 0 the first half, group 1 the second: every chunk once)
    constexpr bool kSU = TB > 0 && EPI == kEpiSwiGLU && LR == 0;
    const bool has_su = kSU && u0 < su;
    const int my_units = my_full + (has_su ? 1 : 0);
    const int su_unit = su_u0 + (u0 >> 1), hs = u0 & 1;
    const int nsteps = P * my_full + (has_su ? P >> 1 : 0);
    // code tiles: 7-bit for codebooks of at most 128 points (TB > 0: known
    // here; TB == 0: per segment, bit g of b7m)
    constexpr bool kB7 = TB > 0 && TB <= 128;
    unsigned b7m = 0;
    if constexpr (TB == 0)
        for (int g = 0; g < a.nseg; g++) b7m |= (unsigned)(kseg[g].n_pts <= 128) << g;
    auto seg_b7 = [&](int g) { return TB > 0 ? kB7 : ((b7m >> g) & 1u) != 0; };
    const uint32_t lof8 = tile_lane_off(false, lane), lof7 = tile_lane_off(true, lane);
    int lk = 0, lj = 0, lts = tile_bytes(kB7);
    uint32_t lof = kB7 ? lof7 : lof8, lso = (uint32_t)(lane & 15);
    int lP = P, lp0 = 0;   // steps of the loaded unit, and its first local chunk
    const unsigned char* lcb = nullptr;
    const uint32_t* lsb = nullptr;
    // half unit: gate and up tiles addressed from the lower of the two
    // bases with a per-lane 32-bit offset (the launcher checks that both
    // tensors lie within 4 GiB of it); lane l loads the word of row
    // 8 hs + (l & 7) of its tensor (l & 8: up), in the lane slot of that row
    auto lset = [&](int k) {
        if (kSU && has_su && min(k, my_units - 1) == my_full) {
            const unsigned char* c0p = reinterpret_cast<const unsigned char*>(kseg[0].codes_t);
            const unsigned char* c1p = reinterpret_cast<const unsigned char*>(kseg[1].codes_t);
            const uint32_t* s0p = kseg[0].scales_t;
            const uint32_t* s1p = kseg[1].scales_t;
            const unsigned char* cb = c0p < c1p ? c0p : c1p;
            const uint32_t* sb = s0p < s1p ? s0p : s1p;
            const bool upl = (lane & 8) != 0;
            const int rl = 8 * hs + (lane & 7);
            lcb = cb + (size_t)su_unit * nc * lts;
            lsb = sb + (size_t)su_unit * nc * 16;
            lof = (uint32_t)((upl ? c1p : c0p) - cb) + tile_lane_off(kB7, (lane & 48) | rl);
            lso = (uint32_t)((upl ? s1p : s0p) - sb) + (uint32_t)rl;
            lP = P >> 1;
            lp0 = grp * (P >> 1);
            return;
        }
        const int uu = min(u0 + min(k, max(my_units - 1, 0)) * nblk, nunits - 1);
        const int g = seg_of(uu);
        const int rb = paired ? uu : uu - ubase(g);
        if constexpr (TB == 0) {
            lts = tile_bytes(seg_b7(g));
            lof = seg_b7(g) ? lof7 : lof8;
        }
        lcb = reinterpret_cast<const unsigned char*>(kseg[g].codes_t) + (size_t)rb * nc * lts;
        lsb = kseg[g].scales_t + (size_t)rb * nc * 16;
    };
    auto lissue = [&](uint4& cw, uint32_t& sw) {
        const int c = wr + (lj + lp0) * WR;
        cw = tile_load(lcb + (size_t)c * lts + lof);
        sw = lsb[c * 16 + lso];
        if (++lj == lP) {
            lj = 0;
            lset(++lk);
        }
    };

    // Each wave stages only its own columns of x (chunks wr + p * WR,
    // p < P) as the MFMA A operand, in a region of LDS no other wave reads:
    // no barrier waits for x, and the weights stream from the first
    // instructions on.  The RMSNorm factor is applied to the finished dot
    // products: y = inv * (W (x * w)), the sums of x^2 of the group's waves
    // meeting in LDS by the first unit end.
    // uniform values that no launch writes while it runs (the position, the
    // codebook fields) are read through the constant address space: scalar
    // loads, which never wait behind the vector loads of the codes
    using KI32 = const __attribute__((address_space(4))) int;
    const int rpos = epi == kEpiRopeKV ? (a.rope.pos_dev ? *(KI32*)a.rope.pos_dev : a.rope.pos) : 0;
    // FA: the tag of this launch's words (token counter * 64 + layer + 1)
    const unsigned fa_tag = FA ? *(KU32*)a.fa.epoch_dev * 64u + (unsigned)a.rope.layer + 1u : 0u;
    uint32_t* X32 = reinterpret_cast<uint32_t*>(dyn + tab_bytes) + (size_t)wid * P * 128;
    const uint4* Xw = reinterpret_cast<const uint4*>(X32);
    // chunks of x per batch of loads (4 when the rank-k rows of three
    // segments come with them: 24 more registers instead of 48)
    constexpr int kXP = kIn && kVS > 2 ? 4 : 8;
    float2 xv[kXP], wv[kXP];
    // LR 1 / 3: the rank-k rows Vt[j] of the wave's columns come with x (slot
    // r of vmask: segment paired ? grp : r / 2, row paired ? r : r % 2), and
    // dk[r] sums x'[c] * Vt[j][c] over them (x' without the RMSNorm factor)
    auto slot_seg = [&](int r) { return paired ? grp : r >> 1; };
    auto slot_row = [&](int r) { return paired ? r : r & 1; };
    unsigned vmask = 0, emask = 0;   // emask: bit 2 g + j, segment g row j, for the epilogue
    if constexpr (kR2) {
        emask = (1u << (2 * a.nseg)) - 1u;
        vmask = paired ? 3u : emask & ((1u << kVS) - 1u);
    } else if constexpr (kIn) {
        // (no short-circuit: seg[0..2] are all in the arguments, and one
        // branch per test would wait for each scalar read in turn)
#pragma unroll
        for (int e = 0; e < 2 * kMaxSeg; e++)
            emask |= (unsigned)(((e >> 1) < a.nseg) & (kseg[e >> 1].tmp_k == nullptr) & (kseg[e >> 1].k > (e & 1))) << e;
        vmask = paired ? (emask >> (2 * grp)) & 3u : emask & ((1u << kVS) - 1u);
    }
    // Vt row of each slot (uniform); an unused slot reads the start of x
    // instead (in bounds: 2 bytes per column against 4), so that the loads
    // are unconditional and go out back to back
    const uint16_t* vrow[kVS];
#pragma unroll
    for (int r = 0; r < kVS; r++) {
        // (LR 3 with a fixed segment count: every slot is used)
        constexpr bool kAll = kR2 && EPI >= 0 && EPI != kEpiStore;
        vrow[r] = kAll || ((vmask >> r) & 1u) ? kseg[slot_seg(r)].Vt + (size_t)slot_row(r) * cols0
                                              : reinterpret_cast<const uint16_t*>(a.x);
    }
    uint32_t vt[kVS][kXP];
    float dk[kVS];
#pragma unroll
    for (int r = 0; r < kVS; r++) dk[r] = 0.f;
    // whole chunks (cols a multiple of 128, every 7B shape) and a norm known
    // here: the loads need no per-lane column test and no fill, and address as
    // a uniform chunk base plus the lane's offset
    const bool whole = kNorm >= 0 && (cols0 & 127) == 0;
    auto xload = [&](int p0) {
        if (whole) {
#pragma unroll
            for (int i = 0; i < kXP; i++) {
                const int p = p0 + i;
                if (p < P) {
                    const int c0 = (wr + p * WR) * 128;
                    xv[i] = *reinterpret_cast<const float2*>(a.x + c0 + 2 * lane);
                    if constexpr (kNorm == 1) wv[i] = *reinterpret_cast<const float2*>(a.norm_w + c0 + 2 * lane);
                    if constexpr (kIn) {
#pragma unroll
                        for (int r = 0; r < kVS; r++) vt[r][i] = *reinterpret_cast<const uint32_t*>(vrow[r] + c0 + 2 * lane);
                    }
                }
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < kXP; i++) {
            const int p = p0 + i, col = (wr + p * WR) * 128 + 2 * lane;
            xv[i] = make_float2(0.f, 0.f);
            wv[i] = make_float2(1.f, 1.f);
#pragma unroll
            for (int r = 0; r < kVS; r++) vt[r][i] = 0u;
            if (p < P && col < a.cols) {
                xv[i] = *reinterpret_cast<const float2*>(a.x + col);
                if (kNorm != 0 && a.norm_w) wv[i] = *reinterpret_cast<const float2*>(a.norm_w + col);
                if constexpr (kIn) {
#pragma unroll
                    for (int r = 0; r < kVS; r++) vt[r][i] = *reinterpret_cast<const uint32_t*>(vrow[r] + col);
                }
            }
        }
    };
    // pair `lane` of local chunk p: (u, v) = (xa wa, xa wa / 2 + xb wb sqrt(3)/2)
    // at dword (((p * 2 + h) * 2 + t) * 4 + g) * 8 + e, and + 4 for the low
    // part (the A-operand order read by step())
    constexpr float kS32 = 0.866025403784438646763723170752936183f;
    const int xoff = ((((lane >> 5) & 1) * 2 + ((lane >> 2) & 1)) * 4 + ((lane >> 3) & 3)) * 8 + (lane & 3);
    float ss = 0.f, mx = 0.f;
    auto xfirst = [&](int p0) {   // fp32 (u, v) in place, sum x^2, max |u|, |v|
#pragma unroll
        for (int i = 0; i < kXP; i++) {
            const int p = p0 + i;
            if (p < P) {
                ss = fmaf(xv[i].x, xv[i].x, ss);
                ss = fmaf(xv[i].y, xv[i].y, ss);
                const float xa = kNorm == 0 ? xv[i].x : xv[i].x * wv[i].x;
                const float xb = kNorm == 0 ? xv[i].y : xv[i].y * wv[i].y;
                if constexpr (kIn) {
                    // every slot, used or not: a loaded word no path consumes
                    // stays pending, and a later reuse of its register then
                    // waits for every load in flight (in the main loop's
                    // header, on every pass)
#pragma unroll
                    for (int r = 0; r < kVS; r++) {
                        dk[r] = fmaf(xa, h2f((uint16_t)(vt[r][i] & 0xFFFFu)), dk[r]);
                        dk[r] = fmaf(xb, h2f((uint16_t)(vt[r][i] >> 16)), dk[r]);
                    }
                }
                const float u = xa, v = fmaf(kS32, xb, 0.5f * xa);
                mx = fmaxf(mx, fmaxf(fabsf(u), fabsf(v)));
                X32[p * 128 + xoff] = __float_as_uint(u);
                X32[p * 128 + xoff + 4] = __float_as_uint(v);
            }
        }
    };

    // this wave's first steps (see the main loop) go out right behind its x:
    // the segment pointers come from scalar loads of the kernel arguments,
    // and vector loads complete in issue order, so the wait for x does not
    // wait for the codes, whose latency overlaps that of x
    xload(0);

    // Epilogue inputs of every unit of the block, loaded now, behind x and
    // ahead of the codes (the wait for x covers them), and kept in LDS.
    // Loaded in the main loop instead, the wait for them at a unit end cannot
    // be counted (the code loads issued in between depend on P), and the
    // compiler's safe count drains most of the loads in flight.  Rank-k
    // factors: one 32-bit load whatever k (k = 2: the fp16 pair; k = 1: the
    // aligned pair holding U[row], half picked at the use; other k: a word
    // of x).  Every loaded register is stored below on every path (a load no
    // path consumes stays pending, and the next use of its register waits
    // for every load in flight).
    constexpr bool kHasPre = EPI == kEpiResidual || EPI < 0, kHasCs = EPI == kEpiRopeKV || EPI < 0;
    float epre[kMv4PreUnits];
    float2 ecs[kMv4PreUnits];
    uint32_t eup[kMv4PreUnits][2];
#pragma unroll
    for (int k = 0; k < kMv4PreUnits; k++) {
        epre[k] = 0.f;
        ecs[k] = make_float2(1.f, 0.f);
        eup[k][0] = eup[k][1] = 0u;
    }
    float esk = 0.f;   // LR 1 / 3: lane 2 g + j of wave 0 holds S[j] of segment g
    if constexpr (kIn) {
        // the three pointers as scalar reads, selected per lane (a per-lane
        // index into the arguments becomes a vector load of the pointer, and
        // the wait for it drains every load in flight); every lane of every
        // wave loads (unused lanes: the start of x), so that no branch merges
        // load sequences of different lengths, after which the compiler
        // drains all loads before the first use of x
        // (global pointers: through a generic one the load would be a flat
        // load, and a flat load in flight makes every later wait a full drain)
        using GF = const __attribute__((address_space(1))) float;
        GF* s0 = (GF*)kseg[0].S;
        GF* s1 = (GF*)kseg[1].S;
        GF* s2 = (GF*)kseg[2].S;
        __asm__ volatile("" : "+s"(s0), "+s"(s1), "+s"(s2));
        const bool use = lane < 2 * kMaxSeg && ((emask >> lane) & 1u);
        GF* sp = !use ? (GF*)a.x : (lane < 2 ? s0 : (lane < 4 ? s1 : s2));
        esk = sp[use ? (lane & 1) : 0];
    }
    if (wid == 0 && lane < 16) {
#pragma unroll
        for (int k = 0; k < kMv4PreUnits; k++) {
            if (k >= my_units) break;
            if (kSU && has_su && k == my_full) break;   // (a half unit has no epilogue inputs)
            const int uu = u0 + k * nblk;
            const int g = seg_of(uu);
            const int prow = (paired ? uu : uu - ubase(g)) * 16 + lane;
            const int r0 = min(prow, kseg[g].rows - 1);
            if (kHasPre && epi == kEpiResidual) epre[k] = a.resid[r0];
            if (kHasCs && epi == kEpiRopeKV) ecs[k] = a.rope.cs[(size_t)rpos * (a.rope.hd >> 1) + ((r0 % a.rope.hd) >> 1)];
#pragma unroll
            for (int gi = 0; gi < 2; gi++) {
                if (LR == 0 || gi >= G) break;
                KSeg& sp = kseg[paired ? gi : g];
                const int kk = kR2 ? 2 : sp.k, r = min(prow, sp.rows - 1);
                const uint32_t* up = kk == 2   ? reinterpret_cast<const uint32_t*>(sp.U) + r
                                     : kk == 1 ? reinterpret_cast<const uint32_t*>(sp.U + (r & ~1))
                                               : reinterpret_cast<const uint32_t*>(a.x);
                eup[k][gi] = *up;
            }
        }
    }

    uint4 cw[DEP];
    uint32_t sw[DEP];
    lset(0);
#pragma unroll
    for (int i = 0; i < DEP; i++) lissue(cw[i], sw[i]);

    // codebook copies: entry e of lane l at byte e * 256 + l * 4.  Wave w
    // writes entries 16w .. 16w + 15 (waves 16 apart when fewer than 16
    // waves cover the table); their fields come in one 64-byte scalar read
    // (the field tables are padded to 256 entries), issued after the code
    // loads: a scalar wait is for every scalar read in flight, so issued
    // earlier it would hold up the reads of the code pointers
    // The residual launches run 8 waves for a single unit per block (o:
    // 4096 x 4096), fewer than the 14 slices of the radius-8 table: there
    // a wave also reads slice wid + 8 in the same round trip (one entry at a
    // time, the remainder took ~11 dependent reads: o 5.66 -> 5.28 us).  Not
    // compiled into the other launches (16 more scalar registers: the head
    // launch ran 4 us slower with them).
    constexpr bool k2S = TB > 128 && EPI == kEpiResidual;
    uint32_t fv[16], fv2[k2S ? 16 : 1];
    const bool two = k2S && NW * 16 < TB && (wid + NW) * 16 < TB;
    if (TB > 0 && wid * 16 < TB) {
        KU32* fp = (KU32*)a.seg[0].fields + wid * 16;
#pragma unroll
        for (int j = 0; j < 16; j++) fv[j] = fp[j];
        if constexpr (k2S) {
            if (two) {
#pragma unroll
                for (int j = 0; j < 16; j++) fv2[j] = fp[NW * 16 + j];
            }
        }
    }
    if (TB > 0) {
        if (wid * 16 < TB) {
#pragma unroll
            for (int j = 0; j < 16; j++) stab[(wid * 16 + j) * 64 + lane] = fv[j];
            if constexpr (k2S) {
                if (two) {
#pragma unroll
                    for (int j = 0; j < 16; j++) stab[((wid + NW) * 16 + j) * 64 + lane] = fv2[j];
                }
            }
        }
        // fewer than TB / 16 waves (TB / 32 with the second slice): the
        // remaining slices, one entry at a time
        KU32* f = (KU32*)a.seg[0].fields;
        for (int e = (k2S ? 2 : 1) * NW * 16 + wid; e < TB; e += NW) stab[e * 64 + lane] = f[e];
    } else {
        for (int g = 0; g < a.nseg; g++) {
            uint32_t* t = reinterpret_cast<uint32_t*>(dyn + toff(g));
            KU32* f = (KU32*)kseg[g].fields;
            for (int e = wid; e < kseg[g].n_pts; e += NW) t[e * 64 + lane] = f[e];
        }
    }
    unsigned have = 0;   // epilogue lanes: rank-k values of segment g fetched
    using KF32 = const __attribute__((address_space(4))) float;
    for (int g = 0; g < (LR == 1 || LR == 2 ? a.nseg : 0); g++) {
        if (kseg[g].k > 0 && kseg[g].tmp_k) {
            for (int j = 0; j < kseg[g].k; j++) {   // uniform index: scalar loads
                const float v = ((KF32*)kseg[g].tmp_k)[j];
                if (wid == 0 && lane == 0) tkl[g][j] = v;
            }
            have |= 1u << g;
        }
    }
    // the only barrier before the first step: the codebook (and tkl)
    lds_barrier();

    xfirst(0);
    if (wid == 0 && lane < 16) {   // x has landed, and with it the epilogue inputs
        if (kIn && lane < 2 * kMaxSeg) lsk[lane] = esk;
#pragma unroll
        for (int k = 0; k < kMv4PreUnits; k++) {
            if constexpr (kHasPre) lpre[k][lane] = epre[k];
            if constexpr (kHasCs) lcs[k][lane] = ecs[k];
            if constexpr (LR > 0) {
                lup[k][0][lane] = eup[k][0];
                lup[k][1][lane] = eup[k][1];
            }
        }
    }
    for (int p0 = kXP; p0 < P; p0 += kXP) {   // more than kXP chunks per wave
        xload(p0);
        xfirst(p0);
    }
    // wave reductions in VALU (DPP and lane swaps): the LDS permutes of
    // shuffles cost 16 waves x 6 steps per value
    ss = wave_sum_valu(ss);
    mx = wave_max_nonneg(mx);   // (fmaxf above keeps NaN out of mx)
    if (lane == 0) ssq[wid] = ss;
    if constexpr (kIn) {
        // the slots' partial sums reduced together: the 32-lane swaps pair
        // slots, the 16-lane swaps put one slot in each 16-lane row, and one
        // DPP row sum finishes them (unused slots hold values nobody reads)
        if constexpr (kVS == 2) {
            const float t = swap_add32(dk[0], dk[1], false);   // lanes 0-31: slot 0, 32-63: slot 1
            const float u = row16_sum(swap_add16(t, t));
            if ((lane & 31) == 0) vtp[lane >> 5][wid] = u;
        } else {
            const float t0 = swap_add32(dk[0], dk[1], false), t1 = swap_add32(dk[2], dk[3], false);
            const float t2 = swap_add32(dk[4], dk[5], false);
            const float u0 = row16_sum(swap_add16(t0, t1));   // rows 0-3: slots 0, 2, 1, 3
            const float u1 = row16_sum(swap_add16(t2, t2));   // rows 0-1: slot 4, rows 2-3: slot 5
            if ((lane & 15) == 0) vtp[((lane >> 4) & 1) * 2 + (lane >> 5)][wid] = u0;
            if ((lane & 31) == 0) vtp[4 + (lane >> 5)][wid] = u1;
        }
    }
    // power-of-two scale putting the wave's largest |u|, |v| near
    // [2^13, 2^14): fp16 high and low parts then hold them to 2^-22
    int ex = 0;
    if (mx > 0.f && mx < INFINITY) (void)frexpf(mx, &ex);
    const float up = ldexpf(1.f, 14 - ex), down = ldexpf(1.f, ex - 14);
    for (int p = 0; p < P; p++) {
        const float uu = __uint_as_float(X32[p * 128 + xoff]) * up;
        const float vv = __uint_as_float(X32[p * 128 + xoff + 4]) * up;
        const _Float16 uh = (_Float16)uu, vh = (_Float16)vv;
        const _Float16 ul = (_Float16)(uu - (float)uh), vl = (_Float16)(vv - (float)vh);
        X32[p * 128 + xoff] = (uint32_t)__builtin_bit_cast(uint16_t, uh) | ((uint32_t)__builtin_bit_cast(uint16_t, vh) << 16);
        X32[p * 128 + xoff + 4] = (uint32_t)__builtin_bit_cast(uint16_t, ul) | ((uint32_t)__builtin_bit_cast(uint16_t, vl) << 16);
    }

    const uint32_t lane_off = (uint32_t)lane * 4u;
    const int m = lane & 15, lg = lane >> 4;
    const uint32_t sh7 = (uint32_t)(lane & 1) * 16u;
    auto step = [&](int g, int p, const uint4 cw, const uint32_t sw, float& acc) {   // local chunk p
        const unsigned char* tb = TB > 0 ? reinterpret_cast<const unsigned char*>(stab) : dyn + toff(g);
        const bool b7 = seg_b7(g);
        uint32_t w4[4] = {cw.x, cw.y, cw.z, cw.w};
        if (b7) align7(w4, sh7);
        // the block scales leave sw before the step's loads are reissued
        // (sw dead early: its next load lands in place instead of in a copy
        // whose move at the loop end would wait for every load in flight)
        float sc[2] = {h2f((uint16_t)(sw & 0xFFFFu)), h2f((uint16_t)(sw >> 16))};
        __asm__ volatile("" : "+v"(sc[0]), "+v"(sc[1]));
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 2; t++) {
                // rows m >= 2 of A only feed rows m >= 2 of D, which are never
                // read: every lane loads row m & 1 (no masking, no zeroing)
                const uint4 xv = Xw[(((p * 2 + h) * 2 + t) * 4 + lg) * 2 + (m & 1)];
                u32x4v aw;
                aw[0] = xv.x; aw[1] = xv.y; aw[2] = xv.z; aw[3] = xv.w;
                u32x4v bw;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t addr = code_addr(w4, 4 * (2 * h + t) + e, lane_off, b7);
                    bw[e] = *reinterpret_cast<const uint32_t*>(tb + addr);
                }
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, aw), __builtin_bit_cast(half8v, bw),
                                                          d, 0, 0, 0);
            }
            acc = fmaf(d[0] + d[1], sc[h], acc);
        }
    };

    int rbuf = 0, uk = 0;   // uk: the block's unit ordinal (epilogue input slot)
    auto unit_end = [&](int u, float& acc, bool half) {
        const int g = seg_of(u);
        if (lane < 16) red[rbuf][wid][lane] = acc * down;
        acc = 0.f;
        lds_barrier();
        if (wid == 0 && lane < 16) {
            // RMSNorm factor of x (gsd_lq_cpu_engine.c:66-82) from the sums of
            // the first group's waves, which cover every column once
            float inv = 1.f;
            if (a.norm_w) {
                float sx = 0.f;
                for (int w = 0; w < WR; w++) sx += ssq[w];
                inv = 1.0f / sqrtf(sx / (float)a.cols + a.eps);
            }
            if constexpr (kIn) {
                // first unit end: rank-k values of the segments without tmp_k,
                // S[j] * inv * (sum of the partials of the waves covering x)
                // (gsd_lq_cpu_engine.c:110-127); lane l reads wave l's partial
                if (!(have & 0x100u)) {
#pragma unroll
                    for (int e = 0; e < 2 * kMaxSeg; e++) {
                        const int r = paired ? (e & 1) : e, w0 = paired ? (e >> 1) * WR : 0;
                        if (r < kVS && ((emask >> e) & 1u)) {
                            // (lanes 0-15 are one DPP row, all active here)
                            const float v = row16_sum(lane < WR ? vtp[r][w0 + lane] : 0.f);
                            tkl[e >> 1][e & 1] = lsk[e] * (v * inv);
                        }
                    }
                    have |= 0x100u;
                }
            }
            if (kSU && half) {
                // half unit: lane l holds row 8 hs + (l & 7) of gate (l < 8)
                // or up (l >= 8), the sum over every wave's own chunks
                float t = 0.f;
                for (int w = 0; w < NW; w++) t += red[rbuf][w][lane];
                t *= inv;
                const int sg = lane >> 3;
                const int row = u * 16 + 8 * hs + (lane & 7);
                if (row < kseg[0].rows) {
                    const uint32_t* rp = sg ? kseg[1].row_ptr : kseg[0].row_ptr;
                    if (rp) {
                        const uint16_t* kcl = sg ? kseg[1].kcols : kseg[0].kcols;
                        const float* kdl = sg ? kseg[1].kdel : kseg[0].kdel;
                        const uint32_t e = rp[row + 1];
                        for (uint32_t i = rp[row]; i < e; i++) t += kdl[i] * xnorm(a, kcl[i], inv);
                    }
                }
                const float upv = __shfl_xor(t, 8, 64);   // lanes 0-7: the up row's value
                if (lane < 8 && row < kseg[0].rows) kseg[0].out[row] = (t / (1.0f + expf(-t))) * upv;
            } else {
                float fin0 = 0.f, fin1 = 0.f;
    #pragma unroll
                for (int gi = 0; gi < 2; gi++) {
                    if (gi >= G) break;
                    const int sg_i = paired ? gi : g;
                    KSeg& sg = kseg[sg_i];
                    const int rb = paired ? u : u - ubase(sg_i);
                    const int row = rb * 16 + lane;
                    float t = 0.f;
                    for (int w = 0; w < WR; w++) t += red[rbuf][gi * WR + w][lane];
                    t *= inv;
                    if (row < sg.rows) {
                        if (sg.row_ptr) {
                            const uint32_t e = sg.row_ptr[row + 1];
                            for (uint32_t i = sg.row_ptr[row]; i < e; i++) t += sg.kdel[i] * xnorm(a, sg.kcols[i], inv);
                        }
                        if (LR > 0 && (kR2 || sg.k > 0)) {
                            if (LR == 2 && !((have >> sg_i) & 1u)) {
                                // bounded wait for the published rank-k words of
                                // this segment (normally already there)
                                int off = 0;
                                for (int g2 = 0; g2 < sg_i; g2++)
                                    if (!a.seg[g2].tmp_k && a.seg[g2].k > 0) off += a.seg[g2].k;
                                int spins = 0;
                                for (int jj = 0; jj < sg.k; jj++) {
                                    unsigned long long wv;
                                    while (((wv = __hip_atomic_load(&a.pub[off + jj], __ATOMIC_RELAXED,
                                                                    __HIP_MEMORY_SCOPE_AGENT)) >> 32) == 0 &&
                                           spins < (1 << 20)) {
                                        if (++spins == (1 << 20)) *a.err = 1u;
                                        __builtin_amdgcn_s_sleep(1);
                                    }
                                    tkl[sg_i][jj] = __uint_as_float((unsigned)wv);
                                }
                                have |= 1u << sg_i;
                            }
                            if (kIn || sg.k <= 2) {   // prefetched factors, same order as below
                                // (the asm keeps the use, and the wait for the
                                // load, inside this branch: hoisted, it would wait
                                // for the code loads in flight in every launch)
                                uint32_t uw = lup[uk][gi][lane];
                                if (!kR2 && sg.k == 1) uw >>= 16 * (row & 1);   // U[row] of the aligned pair
                                t += h2f((uint16_t)(uw & 0xFFFFu)) * tkl[sg_i][0];
                                if (kR2 || sg.k == 2) t += h2f((uint16_t)(uw >> 16)) * tkl[sg_i][1];
                            } else {
                                const uint16_t* up_ = sg.U + (size_t)row * sg.k;
                                for (int jj = 0; jj < sg.k; jj++) t += h2f(up_[jj]) * tkl[sg_i][jj];
                            }
                        }
                    }
                    if (gi == 0) fin0 = t;
                    else fin1 = t;
                }
                KSeg& s0 = kseg[paired ? 0 : g];
                const int row = (paired ? u : u - ubase(g)) * 16 + lane;
                if (paired) {
                    if (row < s0.rows) s0.out[row] = (fin0 / (1.0f + expf(-fin0))) * fin1;
                } else if (epi == kEpiStore) {
                    if (row < s0.rows) s0.out[row] = fin0;
                } else if (epi == kEpiResidual) {
                    if (row < s0.rows) a.resid[row] = lpre[kHasPre ? uk : 0][lane] + fin0;
                } else {
                    // kEpiRopeKV: rows 2i, 2i+1 of a head are one rotation pair
                    // (interleaved RoPE, gsd_lq_cpu_engine.c:213-256) in lanes
                    // 2i, 2i+1; evaluated without contraction like the reference
    #pragma clang fp contract(off)
                    const RopeKV& r = a.rope;
                    const float partner = __shfl_xor(fin0, 1, 64);
                    const size_t base = ((size_t)r.layer * r.max_seq + (size_t)rpos) * (size_t)r.n_kv * r.hd;
                    const bool odd = (lane & 1) != 0;
                    const float x0 = odd ? partner : fin0, x1 = odd ? fin0 : partner;
                    const float2 cs = lcs[kHasCs ? uk : 0][lane];
                    const float y = g == 2 ? fin0 : (odd ? (x0 * cs.y + x1 * cs.x) : (x0 * cs.x - x1 * cs.y));
                    if (row < s0.rows) {
                        if (g == 2) r.v_cache[base + row] = f2h(y);
                        else if (g == 0) s0.out[row] = y;
                        else r.k_cache[base + row] = f2h(y);
                    }
                    if constexpr (FA) {
                        // the same values for the attention blocks: q rows as
                        // fp32, K / V rows as the cache's fp16 pairs (rows 2i,
                        // 2i + 1 in the even lane's word)
                        const uint32_t hp = (uint32_t)f2h(y) | ((uint32_t)f2h(__shfl_xor(y, 1, 64)) << 16);
                        const unsigned long long tag = (unsigned long long)fa_tag << 32;
                        const int qd = r.n_heads * r.hd, kvd = r.n_kv * r.hd;
                        if (row < s0.rows) {
                            if (g == 0)
                                __hip_atomic_store(a.fa.words + row, tag | __float_as_uint(y), __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
                            else if (!odd)
                                __hip_atomic_store(a.fa.words + qd + (g == 2 ? kvd / 2 : 0) + (row >> 1), tag | hp,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
                    }
                }
            }
        }
        rbuf ^= 1;
        uk = min(uk + 1, kMv4PreUnits - 1);   // (the launcher keeps my_units <= kMv4PreUnits)
    };

    float acc = 0.f;
    int cj = 0, ck = 0, cu = u0;
    int cg = seg_of(min(u0, nunits - 1));
    int cP = P, cp0 = 0;   // steps of the computed unit, and its first local chunk
    auto cadvance = [&]() {
        if (++cj == cP) {
            if (ck < my_units) unit_end(cu, acc, kSU && has_su && ck == my_full);
            cj = 0;
            ++ck;
            cu += nblk;
            if (kSU && has_su && ck == my_full) {
                cu = su_unit;
                cP = P >> 1;
                cp0 = grp * (P >> 1);
            }
            cg = seg_of(min(cu, nunits - 1));
        }
    };
    // DEP steps in flight at all times: buffer i holds the steps s
    // with s % DEP == i; every load is issued (the cursor clamps past
    // the end), and the last group may compute steps past the end that no
    // unit end collects
    for (int s = 0; s < nsteps; s += DEP) {
#pragma unroll
        for (int i = 0; i < DEP; i++) {
            step(cg, cj + cp0, cw[i], sw[i], acc);
            lissue(cw[i], sw[i]);
            cadvance();
        }
    }
}

// ------------------------------------------------------------------------
// hexmm: batched projection for prefill (no reference kernel: the reference
// prefills token by token, chat.py:1128-1130).  Same lattice form and tiled
// weight layout as hexmv4; the MFMA A rows are 16 tokens instead of the hi/lo
// parts of one vector:
//   A[m][k] = token m's (u, v) per pair, fp16 after a per-token power-of-two
//             prescale (single rounding: ~1e-4 relative on the outputs),
//   B[k][n] = row n's (r0, r1), decoded once per 128-column chunk and reused
//             for every token group of the block,
//   D lane l = tokens 4(l >> 4) .. +3 of row l & 15.
// A block is 8 waves; wave w owns RBW row-blocks; the block covers TG token
// groups.  Per chunk the A fragments of the block's tokens are staged in LDS
// (loaded into registers one chunk ahead), the codes are double-buffered in
// registers.  Tiles of one row range are placed on one XCD (block b runs on
// XCD b % 8), so their weight reads share that XCD's L2.
// ------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Token row of prep block b of nblocks (one block per row, padded to whole
// 16-token groups): the 16 rows of a group, whose MFMA operand fragments
// interleave in pieces of 4-16 bytes, all on one XCD (blocks go to the 8
// XCDs in turn), so that one L2 assembles each line before writing it back;
// the identity unless the groups divide evenly over the XCDs.
__device__ __forceinline__ int prep_row(int b, int nblocks) {
    if (nblocks & 127) return b;
    const int x = b & 7, j = b >> 3;   // the j-th block on XCD x
    return ((j >> 4) * 8 + x) * 16 + (j & 15);
}

// X bf16 [M][cols] -> A fragments xa[(g16 * nc + c) * 4 + (h * 2 + t)][lane] (uint4
// = (u, v) fp16 of 4 pairs), lane = (m & 15) + 16 * lg, pair 64c + 32h + 8lg + 4t + e;
// xs[m] = the token's descale.  One block per token (padded tokens: zeros).
__global__ void __launch_bounds__(256) hexmm_xprep_kernel(const uint16_t* X, int M, int cols, uint4* xa, float* xs) {
    __shared__ float scratch[16];
    constexpr float kS32 = 0.866025403784438646763723170752936183f;
    const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int nc = (cols + 127) >> 7, np = cols >> 1;
    const bool valid = m < M;
    const uint16_t* xr = X + (size_t)(valid ? m : 0) * cols;
    float mx = 0.f;
    if (valid)
        for (int p = tid; p < np; p += 256) {
            const float xa_ = bf2f(xr[2 * p]), xb_ = bf2f(xr[2 * p + 1]);
            mx = fmaxf(mx, fmaxf(fabsf(xa_), fabsf(fmaf(kS32, xb_, 0.5f * xa_))));
        }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) scratch[wid] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(scratch[0], scratch[1]), fmaxf(scratch[2], scratch[3]));
    int ex = 0;
    if (mx > 0.f && mx < INFINITY) (void)frexpf(mx, &ex);
    const float up = ldexpf(1.f, 14 - ex);
    if (tid == 0) xs[m] = valid ? ldexpf(1.f, ex - 14) : 0.f;
    uint32_t* x32 = reinterpret_cast<uint32_t*>(xa);
    const int g16 = m >> 4, ml = m & 15;
    for (int p = tid; p < nc * 64; p += 256) {
        float u = 0.f, v = 0.f;
        if (valid && p < np) {
            const float xa_ = bf2f(xr[2 * p]), xb_ = bf2f(xr[2 * p + 1]);
            u = xa_ * up;
            v = fmaf(kS32, xb_, 0.5f * xa_) * up;
        }
        const int c = p >> 6, h = (p >> 5) & 1, lg = (p >> 3) & 3, t = (p >> 2) & 1, e = p & 3;
        const size_t idx = ((((size_t)g16 * nc + c) * 4 + h * 2 + t) * 64 + ml + 16 * lg) * 4 + e;
        x32[idx] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)u) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v) << 16);
    }
}

// The same operands for rows of at most 16384 columns from one pass: each
// thread loads its 8-column groups of the row (one 16-byte load each, all in
// flight together), the block finds the largest |u|, |v|, and each group's
// four pairs go out as one 16-byte store.
__global__ void __launch_bounds__(512) hexmm_xprep2_kernel(const uint16_t* X, int M, int cols, uint4* xa, float* xs) {
    __shared__ float red[8];
    constexpr float kS32 = 0.866025403784438646763723170752936183f;
    const int m = prep_row((int)blockIdx.x, (int)gridDim.x), tid = threadIdx.x, wid = tid >> 6;
    const int nc = (cols + 127) >> 7, ng8 = cols >> 3;   // 8-column groups (4 pairs)
    const bool valid = m < M;
    const uint4* xr = reinterpret_cast<const uint4*>(X + (size_t)(valid ? m : 0) * cols);
    uint4 v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = tid + 512 * k;
        v[k] = valid && i < ng8 ? xr[i] : make_uint4(0u, 0u, 0u, 0u);
    }
    auto pair = [](uint32_t w, float& xa_, float& xb_) {
        xa_ = bf2f((uint16_t)(w & 0xFFFFu));
        xb_ = bf2f((uint16_t)(w >> 16));
    };
    float mx = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t w4[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float xa_, xb_;
            pair(w4[e], xa_, xb_);
            mx = fmaxf(mx, fmaxf(fabsf(xa_), fabsf(fmaf(kS32, xb_, 0.5f * xa_))));
        }
    }
    mx = wave_max_nonneg(mx);   // (|x| >= 0; fmaxf above keeps NaN out)
    if ((tid & 63) == 0) red[wid] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < 8; w++) mx = fmaxf(mx, red[w]);
    int ex = 0;
    if (mx > 0.f && mx < INFINITY) (void)frexpf(mx, &ex);
    const float up = ldexpf(1.f, 14 - ex);
    if (tid == 0) xs[m] = valid ? ldexpf(1.f, ex - 14) : 0.f;
    const int g16 = m >> 4, ml = m & 15;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = tid + 512 * k;   // pairs 4 i .. 4 i + 3 (zeros past the row: chunk padding)
        if (i >= nc * 16) continue;
        const int q0 = 4 * i, c = q0 >> 6, h = (q0 >> 5) & 1, lg = (q0 >> 3) & 3, t2 = (q0 >> 2) & 1;
        const uint32_t w4[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float xa_, xb_;
            pair(w4[e], xa_, xb_);
            const float u = xa_ * up, vv = fmaf(kS32, xb_, 0.5f * xa_) * up;
            o[e] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)u) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)vv) << 16);
        }
        xa[(((size_t)g16 * nc + c) * 4 + h * 2 + t2) * 64 + ml + 16 * lg] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

__global__ void __launch_bounds__(256) lowrank_batched_kernel(const uint16_t* X, const uint16_t* Vt, const float* S,
                                                             float* tmp, int k, int cols) {
    __shared__ float scratch[16];
    const int m = blockIdx.x, j = blockIdx.y;
    float p = 0.f;
    for (int c = threadIdx.x; c < cols; c += blockDim.x)
        p = fmaf(bf2f(X[(size_t)m * cols + c]), h2f(Vt[(size_t)j * cols + c]), p);
    p = block_sum(p, scratch);
    if (threadIdx.x == 0) tmp[(size_t)m * k + j] = p * S[j];
}

// Batched operands from fp32 rows (prefill): one block per token (padded
// tokens of the last 16-token group: zero fragments).  x' = (x * inv) * w as
// gsd_lq_cpu_engine.c:66-82, then (u, v) * 2^e as fp16 high and low parts
// at xa[((g16 * nc + c) * 8 + hl * 4 + h * 2 + t) * 64 + (m & 15) + 16 lg]
// (pair 64c + 32h + 8lg + 4t + e, component e of the uint4), and the rank-k
// projections of the tensors that read this input.
__device__ float block_max(float v, float* lds) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    v = wave_max(v);
    __syncthreads();
    if (lane == 0) lds[wid] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < nw; w++) t = fmaxf(t, lds[w]);
    return t;
}

__global__ void __launch_bounds__(256) batch_prep_kernel(const BatchPrep p) {
    __shared__ float scratch[16];
    constexpr float kS32 = 0.866025403784438646763723170752936183f;
    const int m = blockIdx.x, tid = threadIdx.x;
    const int nc = (p.cols + 127) >> 7, np = p.cols >> 1;
    const bool valid = m < p.M;
    const float* xr = p.X + (size_t)(valid ? m : 0) * p.ldx;
    float inv = 1.f;
    if (p.norm_w) {
        float ss = 0.f;
        if (valid)
            for (int c = tid; c < p.cols; c += 256) ss = fmaf(xr[c], xr[c], ss);
        ss = block_sum(ss, scratch);
        inv = 1.0f / sqrtf(ss / (float)p.cols + p.eps);
    }
    auto xprime = [&](int c) { return p.norm_w ? (xr[c] * inv) * p.norm_w[c] : xr[c]; };
    float mx = 0.f;
    if (valid)
        for (int q = tid; q < np; q += 256) {
            const float xa = xprime(2 * q), xb = xprime(2 * q + 1);
            p.xn[(size_t)m * p.cols + 2 * q] = xa;
            p.xn[(size_t)m * p.cols + 2 * q + 1] = xb;
            mx = fmaxf(mx, fmaxf(fabsf(xa), fabsf(fmaf(kS32, xb, 0.5f * xa))));
        }
    mx = block_max(mx, scratch);
    // rank-k projections (block-wide sums in a fixed order)
    for (int g = 0; g < kMaxSeg; g++) {
        for (int j = 0; j < p.k[g]; j++) {
            float d = 0.f;
            if (valid) {
                const uint16_t* vt = p.Vt[g] + (size_t)j * p.cols;
                for (int c = tid; c < p.cols; c += 256) d = fmaf(xprime(c), h2f(vt[c]), d);
            }
            d = block_sum(d, scratch);
            if (valid && tid == 0) p.tmp[g][(size_t)m * p.k[g] + j] = d * p.S[g][j];
        }
    }
    int ex = 0;
    if (mx > 0.f && mx < INFINITY) (void)frexpf(mx, &ex);
    const float up = ldexpf(1.f, 14 - ex);
    if (tid == 0) p.xs[m] = valid ? ldexpf(1.f, ex - 14) : 0.f;
    uint32_t* x32 = reinterpret_cast<uint32_t*>(p.xa);
    const int g16 = m >> 4, ml = m & 15;
    for (int q = tid; q < nc * 64; q += 256) {
        float u = 0.f, v = 0.f;
        if (valid && q < np) {
            const float xa = xprime(2 * q), xb = xprime(2 * q + 1);
            u = xa * up;
            v = fmaf(kS32, xb, 0.5f * xa) * up;
        }
        const _Float16 uh = (_Float16)u, vh = (_Float16)v;
        const _Float16 ul = (_Float16)(u - (float)uh), vl = (_Float16)(v - (float)vh);
        const int c = q >> 6, h = (q >> 5) & 1, lg = (q >> 3) & 3, t = (q >> 2) & 1, e = q & 3;
        const size_t i0 = ((((size_t)g16 * nc + c) * 8 + h * 2 + t) * 64 + ml + 16 * lg) * 4 + e;
        const size_t i1 = i0 + 4 * 64 * 4;   // the low parts: 4 fragments on
        x32[i0] = (uint32_t)__builtin_bit_cast(uint16_t, uh) | ((uint32_t)__builtin_bit_cast(uint16_t, vh) << 16);
        x32[i1] = (uint32_t)__builtin_bit_cast(uint16_t, ul) | ((uint32_t)__builtin_bit_cast(uint16_t, vl) << 16);
    }
}

// The same preparation for inputs of up to kPrep2MaxCols columns and ranks of
// at most 2 per segment, in four passes over the token's row instead of one
// per quantity: the row is read from memory once into LDS (loads in flight
// together), then normed in place, then all rank-k dot products of the
// launch are formed in one pass with one block reduction, then the fp16
// operands are written.  One block of 512 threads per token.
constexpr int kPrep2MaxCols = 32768;
__global__ void __launch_bounds__(512) batch_prep2_kernel(const BatchPrep p) {
    extern __shared__ __attribute__((aligned(16))) float xl[];   // x' of the token [cols]
    __shared__ float red[8][2 * kMaxSeg + 2];
    constexpr float kS32 = 0.866025403784438646763723170752936183f;
    constexpr int NT = 512, NS = 2 * kMaxSeg;
    const int m = prep_row((int)blockIdx.x, (int)gridDim.x), tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int nc = (p.cols + 127) >> 7, np = p.cols >> 1, nv4 = p.cols >> 2;
    const bool valid = m < p.M;
    const float4* xr4 = reinterpret_cast<const float4*>(p.X + (size_t)(valid ? m : 0) * p.ldx);
    float4* xl4 = reinterpret_cast<float4*>(xl);
    auto block_sums = [&](float (&v)[NS + 2], int n) {   // sums over the block of v[0..n)
        for (int s = 0; s < n; s++) {
            const float w = wave_sum_valu(v[s]);
            if (lane == 0) red[wid][s] = w;
        }
        __syncthreads();
        for (int s = 0; s < n; s++) {
            float t = 0.f;
            for (int w = 0; w < NT / 64; w++) t += red[w][s];
            v[s] = t;
        }
        __syncthreads();
    };
    // 1. the row into LDS, and its sum of squares
    float ss = 0.f;
    for (int b = tid; b < nv4; b += 4 * NT) {
        float4 v[4];
#pragma unroll
        for (int k = 0; k < 4; k++)
            v[k] = valid && b + k * NT < nv4 ? xr4[b + k * NT] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (b + k * NT < nv4) {
                xl4[b + k * NT] = v[k];
                ss = fmaf(v[k].x, v[k].x, ss);
                ss = fmaf(v[k].y, v[k].y, ss);
                ss = fmaf(v[k].z, v[k].z, ss);
                ss = fmaf(v[k].w, v[k].w, ss);
            }
        }
    }
    float sv[NS + 2];
    sv[0] = ss;
    block_sums(sv, 1);
    const float inv = p.norm_w ? 1.0f / sqrtf(sv[0] / (float)p.cols + p.eps) : 1.f;
    // 2. x' = (x * inv) * w as the reference forms it, in place; xn; the
    //    largest |u|, |v| (each thread rewrites only its own float4s)
    const float4* w4 = reinterpret_cast<const float4*>(p.norm_w);
    float4* xn4 = reinterpret_cast<float4*>(p.xn + (size_t)m * p.cols);
    float mx = 0.f;
    for (int b = tid; b < nv4; b += 4 * NT) {
        float4 w[4];
#pragma unroll
        for (int k = 0; k < 4; k++)
            w[k] = p.norm_w && b + k * NT < nv4 ? w4[b + k * NT] : make_float4(1.f, 1.f, 1.f, 1.f);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (b + k * NT < nv4) {
                float4 x = xl4[b + k * NT];
                if (p.norm_w) {
                    x.x = (x.x * inv) * w[k].x;
                    x.y = (x.y * inv) * w[k].y;
                    x.z = (x.z * inv) * w[k].z;
                    x.w = (x.w * inv) * w[k].w;
                    xl4[b + k * NT] = x;
                }
                if (valid) xn4[b + k * NT] = x;
                mx = fmaxf(mx, fmaxf(fabsf(x.x), fabsf(fmaf(kS32, x.y, 0.5f * x.x))));
                mx = fmaxf(mx, fmaxf(fabsf(x.z), fabsf(fmaf(kS32, x.w, 0.5f * x.z))));
            }
        }
    }
    // 3. rank-k terms: slot s = 2 g + j (j < k[g] <= 2), x' . Vt[g][j] over
    //    the row, Vt read 4 halves per x' float4
    const uint2* vt[NS];
    bool act[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        act[s] = (s & 1) < p.k[s >> 1];
        vt[s] = act[s] ? reinterpret_cast<const uint2*>(p.Vt[s >> 1] + (size_t)(s & 1) * p.cols) : nullptr;
    }
#pragma unroll
    for (int s = 0; s < NS; s++) sv[s] = 0.f;
    sv[NS] = mx;
    const bool any = act[0] || act[2] || act[4];
    if (valid && any) {
        for (int b = tid; b < nv4; b += 2 * NT) {
            uint2 h[NS][2];
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int k = 0; k < 2; k++) h[s][k] = act[s] && b + k * NT < nv4 ? vt[s][b + k * NT] : make_uint2(0u, 0u);
#pragma unroll
            for (int k = 0; k < 2; k++) {
                if (b + k * NT < nv4) {
                    const float4 x = xl4[b + k * NT];
#pragma unroll
                    for (int s = 0; s < NS; s++) {
                        sv[s] = fmaf(x.x, h2f((uint16_t)(h[s][k].x & 0xFFFFu)), sv[s]);
                        sv[s] = fmaf(x.y, h2f((uint16_t)(h[s][k].x >> 16)), sv[s]);
                        sv[s] = fmaf(x.z, h2f((uint16_t)(h[s][k].y & 0xFFFFu)), sv[s]);
                        sv[s] = fmaf(x.w, h2f((uint16_t)(h[s][k].y >> 16)), sv[s]);
                    }
                }
            }
        }
    }
    // one reduction for the terms (and the max, as a max)
    {
        const float w = wave_max_valu(sv[NS]);
        if (lane == 0) red[wid][NS] = w;
        block_sums(sv, NS);
        float t = 0.f;
        for (int w2 = 0; w2 < NT / 64; w2++) t = fmaxf(t, red[w2][NS]);
        mx = t;
    }
    if (valid && tid < NS && act[tid]) p.tmp[tid >> 1][(size_t)m * p.k[tid >> 1] + (tid & 1)] = sv[tid] * p.S[tid >> 1][tid & 1];
    // 4. (u, v) of x' as fp16 high and low parts after a power-of-two prescale
    int ex = 0;
    if (mx > 0.f && mx < INFINITY) (void)frexpf(mx, &ex);
    const float up = ldexpf(1.f, 14 - ex);
    if (tid == 0) p.xs[m] = valid ? ldexpf(1.f, ex - 14) : 0.f;
    uint32_t* x32 = reinterpret_cast<uint32_t*>(p.xa);
    const int g16 = m >> 4, ml = m & 15;
    for (int q = tid; q < nc * 64; q += NT) {
        float u = 0.f, v = 0.f;
        if (valid && q < np) {
            const float2 x2 = reinterpret_cast<const float2*>(xl)[q];
            u = x2.x * up;
            v = fmaf(kS32, x2.y, 0.5f * x2.x) * up;
        }
        const _Float16 uh = (_Float16)u, vh = (_Float16)v;
        const _Float16 ul = (_Float16)(u - (float)uh), vl = (_Float16)(v - (float)vh);
        const int c = q >> 6, h = (q >> 5) & 1, lg = (q >> 3) & 3, t2 = (q >> 2) & 1, e = q & 3;
        const size_t i0 = ((((size_t)g16 * nc + c) * 8 + h * 2 + t2) * 64 + ml + 16 * lg) * 4 + e;
        const size_t i1 = i0 + 4 * 64 * 4;   // the low parts: 4 fragments on
        x32[i0] = (uint32_t)__builtin_bit_cast(uint16_t, uh) | ((uint32_t)__builtin_bit_cast(uint16_t, vh) << 16);
        x32[i1] = (uint32_t)__builtin_bit_cast(uint16_t, ul) | ((uint32_t)__builtin_bit_cast(uint16_t, vl) << 16);
    }
}

__global__ void __launch_bounds__(256) embed_rows_kernel(const uint16_t* embed, const int* tokens, float* X, int hidden) {
    const int m = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < hidden) X[(size_t)m * hidden + i] = h2f(embed[(size_t)tokens[m] * hidden + i]);
}

// y of one (token, row) of a batched projection: descaled sum, kinks, rank-k
__device__ __forceinline__ float hexmm_finish(const MatmulArgs& a, int m, int row, float s) {
    float y = s * a.xs[m];
    if (a.w.row_ptr) {
        const uint32_t e = a.w.row_ptr[row + 1];
        for (uint32_t j = a.w.row_ptr[row]; j < e; j++)
            y += a.w.kdel[j] * (a.Xf ? a.Xf[(size_t)m * a.cols + a.w.kcols[j]] : bf2f(a.X[(size_t)m * a.cols + a.w.kcols[j]]));
    }
    if (a.w.k > 0)
        for (int j = 0; j < a.w.k; j++) y += h2f(a.w.U[(size_t)row * a.w.k + j]) * a.tmp_k[(size_t)m * a.w.k + j];
    return y;
}

template <int TB, int TG, int RBW, bool HL>
__global__ void __launch_bounds__(512) hexmm_kernel(const MatmulArgs a) {
    constexpr int W = 8;
    constexpr int FPG = HL ? 8 : 4;   // A fragments per token group and chunk
    constexpr int AF = TG * FPG * 64;   // the block's A fragments of one chunk (uint4)
    // two A buffers (one barrier per chunk) for the smaller token tiles (a
    // thread's share of A at most 2 fragments), when they fit beside the
    // codebook; the 8-group tiles measured faster with one buffer and the
    // A fragments one chunk ahead
    constexpr int NAB = (AF + 511) / 512 <= 2 && 2 * AF * 16 + (TB > 0 ? TB * 256 : 0) <= 160 * 1024 ? 2 : 1;
    __shared__ __attribute__((aligned(16))) uint32_t stab[TB > 0 ? TB * 64 : 1];
    __shared__ uint4 As[NAB][AF];
    extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int nc = (a.cols + 127) >> 7;
    const int rows = a.w.rows, nrb = (rows + 15) >> 4, ng = (a.M + 15) >> 4;
    const int n_rt = (nrb + W * RBW - 1) / (W * RBW), n_tt = (ng + TG - 1) / TG;
    const int S = a.nsplit, cps = (nc + S - 1) / S;
    // XCD-aware tile order: the token tiles and column splits of one row
    // tile share XCD b % 8
    const int xcd = (int)blockIdx.x & 7, q = (int)blockIdx.x >> 3;
    const int rt = (q / (n_tt * S)) * 8 + xcd, tt = (q % (n_tt * S)) / S, ks = q % S;
    if (rt >= n_rt) return;
    const int rb0 = rt * W * RBW + wid * RBW;
    const int g0 = tt * TG;
    const int c0 = ks * cps, c1 = min(nc, c0 + cps);
    if (c0 >= c1) return;

    // codes of this wave's row blocks for chunk c (7-bit tiles for
    // codebooks of at most 128 points)
    const bool b7 = TB > 0 ? TB <= 128 : a.w.n_pts <= 128;
    const int tbytes = tile_bytes(b7);
    const uint32_t lof = tile_lane_off(b7, lane), sh7 = (uint32_t)(lane & 1) * 16u;
    const unsigned char* cbase = reinterpret_cast<const unsigned char*>(a.w.codes_t);
    auto load = [&](int c, uint4 (&cw)[RBW], uint32_t (&sw)[RBW]) {
        c = min(c, nc - 1);
#pragma unroll
        for (int r = 0; r < RBW; r++) {
            const size_t i = (size_t)min(rb0 + r, nrb - 1) * nc + c;
            cw[r] = tile_load(cbase + i * tbytes + lof);
            sw[r] = a.w.scales_t[i * 16 + (lane & 15)];
        }
    };
    // this thread's share of the block's A fragments for chunk c
    constexpr int APT = (AF + 511) / 512;
    auto aload = [&](int c, uint4 (&av)[APT]) {
        c = min(c, nc - 1);
#pragma unroll
        for (int i = 0; i < APT; i++) {
            const int j = tid + i * 512;
            const int tg = j / (FPG * 64), g = min(g0 + tg, ng - 1);
            av[i] = j < AF ? a.xa[((size_t)g * nc + c) * (FPG * 64) + (j % (FPG * 64))] : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    // D chunks in flight (A fragments and codes, a ring indexed by the
    // unrolled position): with few MFMAs per chunk a load issued one chunk
    // ahead would leave its whole latency exposed at every chunk
    // (the A fragments one chunk ahead when a thread holds 4 or more)
    constexpr int D = APT <= 1 && RBW <= 1 ? 4 : (APT <= 2 ? 3 : 2);
    constexpr int DA = APT >= 4 ? 1 : D;
    uint4 av[DA][APT];
    uint4 cw[D][RBW];
    uint32_t sw[D][RBW];
#pragma unroll
    for (int i = 0; i < D; i++) {
        if (i < DA) aload(c0 + i, av[i < DA ? i : 0]);
        load(c0 + i, cw[i], sw[i]);
    }

    // codebook: entry e of lane l at byte e * 256 + l * 4
    const int n_pts = a.w.n_pts;
    uint32_t* tabw = TB > 0 ? stab : reinterpret_cast<uint32_t*>(dyn);
    for (int e = wid; e < (TB > 0 ? TB : n_pts); e += W) tabw[e * 64 + lane] = a.w.fields[e];
    const unsigned char* tb = TB > 0 ? reinterpret_cast<const unsigned char*>(stab) : dyn;
    const uint32_t lane_off = (uint32_t)lane * 4u;

    float4v acc[RBW][TG];
#pragma unroll
    for (int r = 0; r < RBW; r++)
#pragma unroll
        for (int g = 0; g < TG; g++) acc[r][g] = float4v{0.f, 0.f, 0.f, 0.f};

    // the shared-codebook kernels decode their one tile format directly; the
    // generic one turns 7-bit words into u8 words first (one decode path)
    constexpr bool B7 = TB > 0 && TB <= 128;
    auto compute = [&](const uint4 (&cw)[RBW], const uint32_t (&sw)[RBW], const uint4* Ab) {
        uint32_t w4[RBW][4];
#pragma unroll
        for (int r = 0; r < RBW; r++) {
            w4[r][0] = cw[r].x; w4[r][1] = cw[r].y; w4[r][2] = cw[r].z; w4[r][3] = cw[r].w;
            if constexpr (B7) align7(w4[r], sh7);
            if constexpr (TB == 0) {
                if (b7) {
                    align7(w4[r], sh7);
                    uint32_t u[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                    for (int j = 0; j < 16; j++) u[j >> 2] |= code_of(w4[r], j, true) << (8 * (j & 3));
#pragma unroll
                    for (int i = 0; i < 4; i++) w4[r][i] = u[i];
                }
            }
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float4v d[RBW][TG];
#pragma unroll
            for (int r = 0; r < RBW; r++)
#pragma unroll
                for (int g = 0; g < TG; g++) d[r][g] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 2; t++) {
                u32x4v bw[RBW];
#pragma unroll
                for (int r = 0; r < RBW; r++) {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        bw[r][e] = *reinterpret_cast<const uint32_t*>(tb + code_addr(w4[r], 4 * (2 * h + t) + e, lane_off, B7));
                }
#pragma unroll
                for (int g = 0; g < TG; g++) {
#pragma unroll
                    for (int hl = 0; hl < (HL ? 2 : 1); hl++) {   // high part, then low part
                        const uint4 xv = Ab[(g * FPG + hl * 4 + h * 2 + t) * 64 + lane];
                        u32x4v aw;
                        aw[0] = xv.x; aw[1] = xv.y; aw[2] = xv.z; aw[3] = xv.w;
#pragma unroll
                        for (int r = 0; r < RBW; r++)
                            d[r][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, aw),
                                                                            __builtin_bit_cast(half8v, bw[r]), d[r][g], 0,
                                                                            0, 0);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < RBW; r++) {
                const float sc = h2f((uint16_t)(h ? (sw[r] >> 16) : (sw[r] & 0xFFFFu)));
#pragma unroll
                for (int g = 0; g < TG; g++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[r][g][i] = fmaf(d[r][g][i], sc, acc[r][g][i]);
            }
        }
    };

    // chunk c: its A fragments go from registers to LDS buffer c % NAB (and
    // the registers reload chunk c + DA), a barrier, the MFMAs; then its
    // code slot reloads chunk c + D (clamped past the end: in bounds,
    // unused).  With two buffers one barrier per
    // chunk suffices: a wave stores buffer b for chunk c + 2 only after the
    // barrier of chunk c + 1, which every wave reaches after its reads of b
    // for chunk c.
    for (int c = c0; c < c1; c += D) {
#pragma unroll
        for (int i = 0; i < D; i++) {
            if (c + i < c1) {
                uint4* Ab = As[NAB == 2 ? (c - c0 + i) & 1 : 0];   // (by chunk parity: D may be odd)
                if (NAB == 1) lds_barrier();
                const int ia = DA == 1 ? 0 : i;
#pragma unroll
                for (int k = 0; k < APT; k++)
                    if (tid + k * 512 < AF) Ab[tid + k * 512] = av[ia][k];
                aload(c + i + DA, av[ia]);
                lds_barrier();
                compute(cw[i], sw[i], Ab);
                load(c + i + D, cw[i], sw[i]);
            }
        }
    }

    // epilogue: token m = 16 (g0 + g) + 4 (lane >> 4) + i, row 16 rb + (lane & 15)
#pragma unroll
    for (int r = 0; r < RBW; r++) {
        const int row = (rb0 + r) * 16 + (lane & 15);
        if (row >= rows) continue;
#pragma unroll
        for (int g = 0; g < TG; g++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = (g0 + g) * 16 + 4 * (lane >> 4) + i;
                if (m >= a.M) continue;
                if (S > 1) {   // partial sum of this column split; hexmm_reduce finishes
                    a.part[((size_t)ks * ng * 16 + m) * rows + row] = acc[r][g][i];
                    continue;
                }
                const float y = hexmm_finish(a, m, row, acc[r][g][i]);
                float* yp = a.Y + (size_t)m * rows + row;
                *yp = a.accumulate ? *yp + y : y;
            }
        }
    }
}

// Column-split partials -> Y: descale, then kinks and rank-k terms (the same
// epilogue as hexmm_kernel); partials summed in split order (deterministic).
__global__ void __launch_bounds__(256) hexmm_reduce_kernel(const MatmulArgs a) {
    const int rows = a.w.rows, ng = (a.M + 15) >> 4;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)a.M * rows) return;
    const int m = (int)(i / rows), row = (int)(i % rows);
    // the partials of 8 splits at a time in flight, summed in split order
    const size_t stride = (size_t)ng * 16 * rows;
    const float* pp = a.part + (size_t)m * rows + row;
    float s = 0.f;
    for (int k0 = 0; k0 < a.nsplit; k0 += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = k0 + k < a.nsplit ? pp[(size_t)(k0 + k) * stride] : 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (k0 + k < a.nsplit) s += v[k];
    }
    const float y = hexmm_finish(a, m, row, s);
    a.Y[i] = a.accumulate ? a.Y[i] + y : y;
}

// ------------------------------------------------------------------------
// Causal attention of a batch of prompt tokens on the matrix cores.  Each
// token computes what the reference's one-token attention computes
// (gsd_lq_cpu_engine.c:264-330; the reference prefills token by token,
// run_gpu_native_chat.py:1128-1130): token t of the batch sits at position
// p0 + t and attends over cache positions 0 .. p0 + t.
// Block: KV head blockIdx.y and 64 query rows, T = 64 / G consecutive tokens
// x the G query heads of the KV head (row r: token t0 + r / G, head
// kvh * G + r % G); wave w holds rows 16w .. 16w + 15, one per lane column
// (lane & 15).  Positions pass through LDS in chunks of 32, K as rows
// [pos][HD] and V transposed [HD][pos] (rows padded against bank conflicts),
// double-buffered with the next chunk's loads in flight.  Per chunk a wave
// forms S^T = K Q^T (two 16-position tiles; A: K rows, B: the lane's query
// row as fp16 high + low parts after a per-row power-of-two scale, so the
// scores keep ~22 bits), the online softmax of each query row (base-2
// exponent: the scale carries log2 e), and O^T += V^T P^T (A: V^T, B: the
// probabilities, high + low parts).  The k index of the second product runs
// over the chunk's positions in the order the score tiles leave them in a
// lane of group g = lane >> 4 (4g .. 4g+3, then 16+4g .. 16+4g+3), and the
// V^T fragments are read in that order.  Positions past the block's last
// token are staged as zeros: cache rows past the context may hold anything,
// and a zero probability times a NaN would still be NaN.
template <int HD>
__global__ void __launch_bounds__(256) attn_prefill_kernel(const PrefillAttn a) {
    constexpr int KS = HD + 8;    // K row stride, halves (16 bytes of padding)
    constexpr int VS = 36;        // V^T row stride, halves (32 positions + 4)
    constexpr int NKS = HD / 32;  // k steps of the scores
    constexpr int NDT = HD / 16;  // 16-dimension tiles of the output
    constexpr int D8 = HD / 8;    // 16-byte pieces of a cache row
    constexpr int NK = HD / 64;   // K pieces per thread and chunk (32 * D8 / 256)
    constexpr int NVU = 16 * D8;  // V units: 16 position pairs x D8 pieces
    constexpr int NV = (NVU + 255) / 256;
    __shared__ __attribute__((aligned(16))) uint16_t kl[2][32 * KS];
    __shared__ __attribute__((aligned(16))) uint16_t vl[2][HD * VS];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int lg = a.log2g, G = 1 << lg, T = 64 >> lg;
    const int grp = (int)gridDim.x - 1 - (int)blockIdx.x;   // the longest blocks first
    const int kvh = (int)blockIdx.y;
    const int t0 = grp * T;
    const int r = 16 * wid + n;
    const int t = t0 + (r >> lg), head = kvh * G + (r & (G - 1));
    const bool valid = t < a.M;
    const int limit = a.p0 + t;   // last position of this row
    const int maxpos = a.p0 + min(t0 + T, a.M) - 1;
    const int nch = maxpos / 32 + 1;

    // the row's query: B fragments of k step ks = dims 32 ks + 8 g .. + 7
    half8v qh[NKS], ql[NKS];
    float down;
    {
        const float qs = a.sm_scale * 1.44269504088896340736f;
        const float* qr = a.q + ((size_t)(valid ? t : 0) * a.n_heads + head) * HD + 8 * g;
        float qv[NKS][8];
        float mx = 0.f;
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) {
            float4 f0 = make_float4(0.f, 0.f, 0.f, 0.f), f1 = f0;
            if (valid) {
                f0 = *reinterpret_cast<const float4*>(qr + 32 * ks);
                f1 = *reinterpret_cast<const float4*>(qr + 32 * ks + 4);
            }
            const float v8[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                qv[ks][j] = v8[j] * qs;
                mx = fmaxf(mx, fabsf(qv[ks][j]));
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        int ex = 0;
        if (mx > 0.f && mx < INFINITY) (void)frexpf(mx, &ex);
        const float up = ldexpf(1.f, 14 - ex);
        down = ldexpf(1.f, ex - 14);
#pragma unroll
        for (int ks = 0; ks < NKS; ks++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float x = qv[ks][j] * up;
                const _Float16 h = (_Float16)x;
                qh[ks][j] = h;
                ql[ks][j] = (_Float16)(x - (float)h);
            }
    }

    const size_t rstride = (size_t)a.n_kv * HD;   // halves from one position to the next
    const size_t lbase = ((size_t)a.layer * a.max_seq * a.n_kv + kvh) * HD;
    const uint16_t* kbase = a.k_cache + lbase;
    const uint16_t* vbase = a.v_cache + lbase;
    uint4 kr[NK], vr[NV][2];
    const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
    auto fetch = [&](int c) {
        const int c0 = 32 * c;
#pragma unroll
        for (int i = 0; i < NK; i++) {
            const int idx = tid + 256 * i, p = c0 + idx / D8;
            kr[i] = p <= maxpos ? *reinterpret_cast<const uint4*>(kbase + (size_t)p * rstride + (idx % D8) * 8) : z4;
        }
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int idx = tid + 256 * i, p = c0 + 2 * (idx / D8);
            const bool ok = idx < NVU;
            const size_t off = (size_t)p * rstride + (idx % D8) * 8;
            vr[i][0] = ok && p <= maxpos ? *reinterpret_cast<const uint4*>(vbase + off) : z4;
            vr[i][1] = ok && p + 1 <= maxpos ? *reinterpret_cast<const uint4*>(vbase + off + rstride) : z4;
        }
    };
    auto put = [&](int b) {
#pragma unroll
        for (int i = 0; i < NK; i++) {
            const int idx = tid + 256 * i;
            *reinterpret_cast<uint4*>(&kl[b][(idx / D8) * KS + (idx % D8) * 8]) = kr[i];
        }
        uint32_t* vw = reinterpret_cast<uint32_t*>(&vl[b][0]);
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int idx = tid + 256 * i;
            if (idx < NVU) {
                const int j = idx / D8, d0 = (idx % D8) * 8;
                const uint32_t e0[4] = {vr[i][0].x, vr[i][0].y, vr[i][0].z, vr[i][0].w};
                const uint32_t e1[4] = {vr[i][1].x, vr[i][1].y, vr[i][1].z, vr[i][1].w};
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const uint32_t lo = (e0[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
                    const uint32_t hi = (e1[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
                    vw[((d0 + e) * VS) / 2 + j] = lo | (hi << 16);
                }
            }
        }
    };

    float4v o[NDT];
#pragma unroll
    for (int d = 0; d < NDT; d++) o[d] = float4v{0.f, 0.f, 0.f, 0.f};
    float mrun = -INFINITY, lsum = 0.f;
    fetch(0);
    put(0);
    __syncthreads();
    for (int c = 0; c < nch; c++) {
        if (c + 1 < nch) fetch(c + 1);
        const uint16_t* kb = kl[c & 1];
        const uint16_t* vb = vl[c & 1];
        float4v sa = {0.f, 0.f, 0.f, 0.f}, sb = sa;
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) {
            const half8v ka = *reinterpret_cast<const half8v*>(kb + n * KS + 32 * ks + 8 * g);
            const half8v kb2 = *reinterpret_cast<const half8v*>(kb + (16 + n) * KS + 32 * ks + 8 * g);
            sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[ks], sa, 0, 0, 0);
            sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[ks], sa, 0, 0, 0);
            sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb2, qh[ks], sb, 0, 0, 0);
            sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb2, ql[ks], sb, 0, 0, 0);
        }
        // lane: positions c0 + 4g + i (tile a) and c0 + 16 + 4g + i (tile b) of row n
        const int pa = 32 * c + 4 * g;
        float s[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s[i] = pa + i <= limit ? sa[i] * down : -INFINITY;
            s[4 + i] = pa + 16 + i <= limit ? sb[i] * down : -INFINITY;
        }
        float mc = s[0];
#pragma unroll
        for (int i = 1; i < 8; i++) mc = fmaxf(mc, s[i]);
        mc = fmaxf(mc, __shfl_xor(mc, 16, 64));
        mc = fmaxf(mc, __shfl_xor(mc, 32, 64));
        // position 0 is in every row's range, so the running maximum is
        // finite from the first chunk on (alpha = 0 there)
        const float mnew = fmaxf(mrun, mc);
        const float alpha = exp2f(mrun - mnew);
        mrun = mnew;
        half8v ph, pl;
        float ps = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float pj = exp2f(s[j] - mnew);
            ps += pj;
            const _Float16 h = (_Float16)pj;
            ph[j] = h;
            pl[j] = (_Float16)(pj - (float)h);
        }
        lsum = lsum * alpha + ps;
#pragma unroll
        for (int d = 0; d < NDT; d++) {
            o[d] *= alpha;
            const uint16_t* vrow = vb + (d * 16 + n) * VS;
            const uint2 lo4 = *reinterpret_cast<const uint2*>(vrow + 4 * g);
            const uint2 hi4 = *reinterpret_cast<const uint2*>(vrow + 16 + 4 * g);
            const u32x4v vw = {lo4.x, lo4.y, hi4.x, hi4.y};
            const half8v va = __builtin_bit_cast(half8v, vw);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph, o[d], 0, 0, 0);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, o[d], 0, 0, 0);
        }
        if (c + 1 < nch) put((c + 1) & 1);
        __syncthreads();
    }
    float l = lsum + __shfl_xor(lsum, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (valid) {
        const float inv = 1.0f / l;
        float* out = a.out + ((size_t)t * a.n_heads + head) * HD + 4 * g;
#pragma unroll
        for (int d = 0; d < NDT; d++)
            *reinterpret_cast<float4*>(out + 16 * d) = make_float4(o[d][0] * inv, o[d][1] * inv, o[d][2] * inv, o[d][3] * inv);
    }
}

}  // namespace

// ------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------
hipError_t launch_hexmv(const HexArgs& a, hipStream_t st) {
    const int S = a.cols >> 5;
    // one 32-column slot per thread (fewest VGPRs, most waves per CU); two
    // when the row has more than 1024 slots
    const int spt = S <= 1024 ? 1 : 2;
    const int nt = ((S + spt - 1) / spt + 63) / 64 * 64;
    if (nt > 1024) return hipErrorInvalidValue;
    bool lattice = a.nseg > 0, shared = true;
    for (int g = 0; g < a.nseg; g++) {
        lattice = lattice && a.seg[g].fields != nullptr;
        shared = shared && a.seg[g].fields == a.seg[0].fields && a.seg[g].n_pts == a.seg[0].n_pts;
    }
    // lattice fields come with the 4-row scale groups; the generic path
    // reads the file's row-major scales
    if (lattice != (a.scale_t != 0)) return hipErrorInvalidValue;
#define GSD_HEXMV_DISPATCH(ST, TM)                                                  \
    if (spt == 2) {                                                                 \
        if (nt <= 64) return launch_hexmv_t<2, 1, ST, TM>(a, st, nt);                \
        if (nt <= 256) return launch_hexmv_t<2, 4, ST, TM>(a, st, nt);               \
        if (nt <= 512) return launch_hexmv_t<2, 8, ST, TM>(a, st, nt);               \
        return launch_hexmv_t<2, 16, ST, TM>(a, st, nt);                             \
    }                                                                               \
    if (nt <= 64) return launch_hexmv_t<1, 1, ST, TM>(a, st, nt);                    \
    if (nt <= 256) return launch_hexmv_t<1, 4, ST, TM>(a, st, nt);                   \
    if (nt <= 512) return launch_hexmv_t<1, 8, ST, TM>(a, st, nt);                   \
    return launch_hexmv_t<1, 16, ST, TM>(a, st, nt);
    if (!lattice) {
        GSD_HEXMV_DISPATCH(false, 0)
    } else if (shared) {
        GSD_HEXMV_DISPATCH(true, 1)
    } else {
        GSD_HEXMV_DISPATCH(true, 2)
    }
#undef GSD_HEXMV_DISPATCH
}

// Half units of a paired launch (GSD_GATEUP_HALVES=0 turns them off, to
// compare the two plans), and whether gate's and up's tiles and scales lie
// within 4 GiB of the lower base, as the kernel's 32-bit lane offsets need.
static bool half_units_on() {
    const char* e = std::getenv("GSD_GATEUP_HALVES");
    return !(e && e[0] == '0');
}
static bool half_units_reach(const HexArgs& a) {
    const HexSeg &g = a.seg[0], &u = a.seg[1];
    const uint64_t nrb = (uint64_t)(g.rows + 15) / 16, nc = (uint64_t)(a.cols + 127) / 128;
    const uint64_t tb = g.n_pts <= 128 ? kTile7 : kTileU8;
    auto span = [](uint64_t p, uint64_t q, uint64_t n) { return (p > q ? p : q) + n - (p < q ? p : q); };
    return span((uint64_t)(uintptr_t)g.codes_t, (uint64_t)(uintptr_t)u.codes_t, nrb * nc * tb) < (1ull << 32) &&
           span((uint64_t)(uintptr_t)g.scales_t, (uint64_t)(uintptr_t)u.scales_t, nrb * nc * 64) < (1ull << 32);
}

template <int TB, int LR, int EPI, int DEP = kMv4Depth>
hipError_t launch_hexmv4_t(const HexArgs& a0, hipStream_t st, int nw, size_t lds, int nunits, int nlead) {
    static int per_cu = 0;
    static size_t attr_lds = 0;
    if (lds > attr_lds) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&hexmv4_kernel<TB, LR, EPI, 0, 0, DEP>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_lds = lds;
        per_cu = 0;
    }
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, hexmv4_kernel<TB, LR, EPI, 0, 0, DEP>, nw * 64, lds) != hipSuccess ||
        n < 1)
        return hipErrorInvalidConfiguration;
    per_cu = n;
    const int ncu = device_cu_count() > 0 ? device_cu_count() : 256;
    // publishing blocks (LR == 2) first (dispatched in order, they are
    // resident before any matvec block waits on them), and all blocks
    // resident at once
    int grid = ncu * per_cu - nlead;
    if (grid < 1) grid = 1;
    if (grid > nunits) grid = nunits;
    // at most kMv4PreUnits units per block (more blocks than fit at once
    // beyond 8 units per CU: the later ones start as earlier ones finish)
    if (grid < (nunits + kMv4PreUnits - 1) / kMv4PreUnits) grid = (nunits + kMv4PreUnits - 1) / kMv4PreUnits;
    HexArgs a = a0;
    a.mv.units_q = nunits / grid;
    a.mv.units_r = nunits % grid;
    a.mv.su = 0;
    a.mv.su_u0 = 0;
    if constexpr (TB > 0 && EPI == kEpiSwiGLU && LR == 0) {
        // the last, partial round of units as half units on twice the
        // blocks (gate/up 7B: 896 units on 256 blocks, 3.5 each)
        const int R = nunits % grid;
        if (R > 0 && 2 * R <= grid && a.mv.P % 2 == 0 && half_units_on() && half_units_reach(a)) {
            a.mv.units_r = 0;
            a.mv.su = 2 * R;
            a.mv.su_u0 = a.mv.units_q * grid;
        }
    }
    hipLaunchKernelGGL((hexmv4_kernel<TB, LR, EPI, 0, 0, DEP>), dim3(grid + nlead), dim3(nw * 64), lds, st, a);
    return hipGetLastError();
}

// q/k/v + decode attention (hexmv4_kernel with FAHD > 0): matvec blocks first, then one
// attention block per KV head, all resident at once (the attention blocks
// wait for words of matvec blocks); blocks of max(nw, 8) waves (the
// attention runs 8).  hipErrorNotSupported before any launch when that does
// not fit.
template <int TB, int LR, int HD, int G, int PW>
hipError_t launch_qkva_t(const HexArgs& a0, hipStream_t st, int nw, size_t lds, int nunits) {
    const int nt = (nw > 8 ? nw : 8) * 64;
    static size_t attr_lds = 0;
    if (lds > attr_lds) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&hexmv4_kernel<TB, LR, kEpiRopeKV, HD, G, kMv4Depth, PW>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_lds = lds;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, hexmv4_kernel<TB, LR, kEpiRopeKV, HD, G, kMv4Depth, PW>, nt, lds) != hipSuccess || per_cu < 1)
        return hipErrorNotSupported;
    const int ncu = device_cu_count() > 0 ? device_cu_count() : 256;
    int grid = ncu * per_cu - a0.fa.nkv;   // matvec blocks
    if (grid > nunits) grid = nunits;
    if (grid < 1 || grid < (nunits + kMv4PreUnits - 1) / kMv4PreUnits) return hipErrorNotSupported;
    HexArgs a = a0;
    a.mv.units_q = nunits / grid;
    a.mv.units_r = nunits % grid;
    a.mv.nw = nw;
    hipLaunchKernelGGL((hexmv4_kernel<TB, LR, kEpiRopeKV, HD, G, kMv4Depth, PW>), dim3(grid + a.fa.nkv), dim3(nt), lds, st, a);
    return hipGetLastError();
}

hipError_t launch_hexmv4(const HexArgs& a, hipStream_t st) {
    if (a.nseg < 1 || a.nseg > kMaxSeg || a.cols <= 0 || a.cols % 64) return hipErrorInvalidValue;
    const int nc = (a.cols + 127) / 128;
    const bool paired = a.epilogue == kEpiSwiGLU;
    if (paired && (a.nseg != 2 || a.seg[0].rows != a.seg[1].rows)) return hipErrorInvalidValue;
    if (a.epilogue == kEpiRopeKV && a.nseg != 3) return hipErrorInvalidValue;
    bool shared = true, lr = false, inblock = a.epilogue != kEpiResidual || a.nseg == 1, all2 = true;
    int nlead = 0, nunits = 0, tab_bytes = 0;
    for (int g = 0; g < a.nseg; g++) {
        const HexSeg& s = a.seg[g];
        if (!s.codes_t || !s.scales_t || !s.fields || s.n_pts < 1 || s.n_pts > kTableSlots) return hipErrorInvalidValue;
        shared = shared && s.fields == a.seg[0].fields && s.n_pts == a.seg[0].n_pts;
        if (s.k > 0 && (!s.U || (!s.tmp_k && (!s.Vt || !s.S)))) return hipErrorInvalidValue;
        lr = lr || s.k > 0;
        all2 = all2 && s.k == 2 && !s.tmp_k;
        if (!s.tmp_k && s.k > 0) {
            nlead += s.k;
            inblock = inblock && s.k <= 2;
        }
        nunits += (s.rows + 15) / 16;
        tab_bytes += s.n_pts * 256;
    }
    if (paired) nunits = (a.seg[0].rows + 15) / 16;
    // ranks <= 2 (every model tensor of the Precision mode): each block forms
    // the projections from its own staging of x; otherwise leading blocks
    // publish them (generic epilogue)
    if (inblock) nlead = 0;
    if (nlead > 0 && (!a.pub || !a.err)) return hipErrorInvalidValue;
    if (nunits == 0) return hipSuccess;
    // waves per row-block: up to 16 (8 per group when paired), at most one
    // per 128-column chunk
    // waves per row-block: the largest power of two <= 16 / G dividing the
    // chunk count (so every wave has the same number of chunks per unit)
    const int G = paired ? 2 : 1;
    // 8 waves instead of 16 when every block has one unit and the wave's
    // chunks still fit one batch of x loads (o: 4096 x 4096): the prologue,
    // which every wave runs and four waves per SIMD issue in turn, then
    // reaches the code loads sooner (measured: o 7.6 -> 6.7 us); two units or
    // more per block (q/k/v) measured slower, and so did down with 8 waves
    // and all its x in one batch (8 waves x 4 steps hold half the bytes in
    // flight that a 31 MB launch needs at the HBM rate)
    const bool few = nunits <= device_cu_count() && nc <= 64;
    int wr = (few ? kMv4MaxWaves / 2 : kMv4MaxWaves) / G, wr_log2 = (few ? 3 : 4) - (G - 1);
    while (wr > 1 && nc % wr != 0) {
        wr >>= 1;
        wr_log2--;
    }
    const int nw = wr * G;
    HexArgs ap = a;   // with the launch plan
    ap.mv.P = nc / wr;
    ap.mv.wr_log2 = wr_log2;
    ap.mv.nunits = nunits;
    ap.mv.ub1 = (a.seg[0].rows + 15) / 16;
    ap.mv.ub2 = ap.mv.ub1 + (a.nseg > 1 ? (a.seg[1].rows + 15) / 16 : 0);
    const size_t xbytes = (size_t)G * nc * 512;   // every wave's own chunks of x
    ap.mv.nw = nw;
    if (a.fa.nkv > 0) {
        // the q/k/v launch with the decode attention in its last blocks
        const int gq = a.rope.n_kv > 0 ? a.rope.n_heads / a.rope.n_kv : 0;
        const int lrm = !lr ? 0 : (inblock && all2 ? 3 : -1);
        if (a.epilogue != kEpiRopeKV || !shared || !a.norm_w || !a.fa.words || !a.fa.out || !a.fa.epoch_dev ||
            !a.rope.pos_dev || a.fa.nkv != a.rope.n_kv || gq * a.rope.n_kv != a.rope.n_heads || a.rope.layer < 0 ||
            a.rope.layer >= 64)
            return hipErrorNotSupported;
#define GSD_QAP(T, L, HD, G)                                                                                    \
    {                                                                                                           \
        if (a.fa.span == 64) return launch_qkva_t<T, L, HD, G, 8>(ap, st, nw, xbytes, nunits);                  \
        if (a.fa.span == 128) return launch_qkva_t<T, L, HD, G, 16>(ap, st, nw, xbytes, nunits);                \
        return launch_qkva_t<T, L, HD, G, 32>(ap, st, nw, xbytes, nunits);                                      \
    }
#define GSD_QA(T, L)                                                                                            \
    {                                                                                                           \
        if (a.rope.hd == 128 && gq == 4) GSD_QAP(T, L, 128, 4)                                                  \
        if (a.rope.hd == 64 && gq == 2) GSD_QAP(T, L, 64, 2)                                                    \
        return hipErrorNotSupported;                                                                            \
    }
        if (a.seg[0].n_pts == 217 && lrm == 0) GSD_QA(217, 0)
        if (a.seg[0].n_pts == 217 && lrm == 3) GSD_QA(217, 3)
        if (a.seg[0].n_pts == 127 && lrm == 0) GSD_QA(127, 0)
        if (a.seg[0].n_pts == 127 && lrm == 3) GSD_QA(127, 3)
#undef GSD_QA
#undef GSD_QAP
        return hipErrorNotSupported;
    }
    // the shared-codebook kernels are specialised on the epilogue as well.
    // Many units per block (the output projection: 2048 units on 256 CUs)
    // stream at a ring depth of 4: at 2, each CU's 16 waves keep 32 KB in
    // flight, which at the memory latency is about half the HBM rate
    const bool deep = nunits >= 6 * (device_cu_count() > 0 ? device_cu_count() : 256);
#define GSD_MV4(T, E)                                                                           \
    {                                                                                           \
        const size_t lds = xbytes + (T == 0 ? (size_t)tab_bytes : 0);                           \
        if constexpr (T > 0 && E == kEpiStore) {                                                \
            if (deep && !lr) return launch_hexmv4_t<T, 0, E, 4>(ap, st, nw, lds, nunits, 0);     \
            if (deep && inblock && all2) return launch_hexmv4_t<T, 3, E, 4>(ap, st, nw, lds, nunits, 0); \
        }                                                                                       \
        if (!lr) return launch_hexmv4_t<T, 0, E>(ap, st, nw, lds, nunits, 0);                   \
        if (inblock && all2) return launch_hexmv4_t<T, 3, E>(ap, st, nw, lds, nunits, 0);       \
        if (inblock) return launch_hexmv4_t<T, 1, E>(ap, st, nw, lds, nunits, 0);               \
        return launch_hexmv4_t<T, 2, -1>(ap, st, nw, lds, nunits, nlead);                       \
    }
#define GSD_MV4E(T)                                          \
    switch (a.epilogue) {                                    \
        case kEpiStore: GSD_MV4(T, kEpiStore)                \
        case kEpiResidual: GSD_MV4(T, kEpiResidual)          \
        case kEpiSwiGLU: GSD_MV4(T, kEpiSwiGLU)              \
        case kEpiRopeKV: GSD_MV4(T, kEpiRopeKV)              \
        default: return hipErrorInvalidValue;                \
    }
    // the epilogue-specialised kernels fix the RMSNorm by the epilogue (with
    // it: RoPE + K/V append and SwiGLU; without it: residual)
    const bool norm_fixed = a.epilogue == kEpiResidual ? a.norm_w == nullptr
                            : (a.epilogue == kEpiSwiGLU || a.epilogue == kEpiRopeKV) ? a.norm_w != nullptr
                                                                                      : true;
    if (shared && norm_fixed && a.seg[0].n_pts == 217) GSD_MV4E(217)
    if (shared && norm_fixed && a.seg[0].n_pts == 127) GSD_MV4E(127)
    GSD_MV4(0, -1)
#undef GSD_MV4E
#undef GSD_MV4
}

size_t hexmm_xa_bytes(int M, int cols, int hl) {
    const size_t ng = ((size_t)M + 15) / 16, nc = ((size_t)cols + 127) / 128;
    return ng * nc * (hl ? 8 : 4) * 64 * 16;
}

template <int TB, int TG, int RBW, bool HL>
hipError_t launch_hexmm_t(const MatmulArgs& a, hipStream_t st) {
    const int nrb = (a.w.rows + 15) / 16, ng = (a.M + 15) / 16;
    const int n_rt = (nrb + 8 * RBW - 1) / (8 * RBW), n_tt = (ng + TG - 1) / TG;
    const int grid = 8 * n_tt * a.nsplit * ((n_rt + 7) / 8);
    const size_t lds = TB > 0 ? 0 : (size_t)a.w.n_pts * 256;
    if (lds > 0) {
        static size_t attr = 0;
        if (lds > attr) {
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&hexmm_kernel<TB, TG, RBW, HL>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
            attr = lds;
        }
    }
    hipLaunchKernelGGL((hexmm_kernel<TB, TG, RBW, HL>), dim3(grid), dim3(512), lds, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit <= 1) return e;
    const size_t n = (size_t)a.M * a.w.rows;
    hipLaunchKernelGGL(hexmm_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a);
    return hipGetLastError();
}

MatmulPlan hexmm_plan(int M, int rows, int cols, bool hl) {
    // fewest token tiles (largest tg: the weights are decoded once per token
    // tile) that still give about 3/4 of a block per CU; when no tiling does,
    // split the columns (at least 4 chunks per split, partials within twice
    // the code bytes)
    const int nc = (cols + 127) / 128, nrb = (rows + 15) / 16, ng = (M + 15) / 16;
    const int ncu = device_cu_count() > 0 ? device_cu_count() : 256;
    MatmulPlan p{1, 1, 1};
    int tiles = 0;
    // high + low operands (two matrix-core products per step) from 256
    // tokens on: the eight-group tile, its columns split until the grid
    // fills the chip, where the rule below would take fewer token groups
    // per tile (7B prompt of 1024 tokens: 54.4 -> 51.1 ms; the single-
    // operand projection measured 3 % slower this way)
    if (hl && ng >= 16) {
        const int t8 = ((nrb + 15) / 16) * ((ng + 7) / 8);
        if (4 * t8 < 3 * ncu) {
            const int s = std::min((ncu + t8 - 1) / t8, std::max(1, nc / 4));
            return MatmulPlan{8, 2, s};
        }
    }
    for (int tg = 8; tg >= 1; tg >>= 1) {
        if (tg > 1 && tg > ng) continue;
        const int rbw = tg == 8 ? 2 : 1;
        tiles = ((nrb + 8 * rbw - 1) / (8 * rbw)) * ((ng + tg - 1) / tg);
        p = MatmulPlan{tg, rbw, 1};
        if (4 * tiles >= 3 * ncu) return p;
    }
    int s = (2 * ncu + tiles - 1) / tiles;
    s = std::min(s, std::max(1, nc / 4));
    const long long cap = ((long long)rows * cols) / (4LL * (ng * 16) * rows);
    p.nsplit = (int)std::max<long long>(1, std::min<long long>(s, cap));
    return p;
}

template <int TB>
hipError_t launch_hexmm_tb(const MatmulArgs& a, hipStream_t st) {
    if (a.hl) {
        if (a.tg == 8 && a.rbw == 2) return launch_hexmm_t<TB, 8, 2, true>(a, st);
        if (a.tg == 4 && a.rbw == 1) return launch_hexmm_t<TB, 4, 1, true>(a, st);
        if (a.tg == 2 && a.rbw == 1) return launch_hexmm_t<TB, 2, 1, true>(a, st);
        if (a.tg == 1 && a.rbw == 1) return launch_hexmm_t<TB, 1, 1, true>(a, st);
        return hipErrorInvalidValue;
    }
    if (a.tg == 8 && a.rbw == 2) return launch_hexmm_t<TB, 8, 2, false>(a, st);
    if (a.tg == 4 && a.rbw == 1) return launch_hexmm_t<TB, 4, 1, false>(a, st);
    if (a.tg == 2 && a.rbw == 1) return launch_hexmm_t<TB, 2, 1, false>(a, st);
    if (a.tg == 1 && a.rbw == 1) return launch_hexmm_t<TB, 1, 1, false>(a, st);
    return hipErrorInvalidValue;
}

hipError_t launch_hexmm_prepared(const MatmulArgs& a, hipStream_t st) {
    if (a.M <= 0 || a.cols <= 0 || a.cols % 64 || !a.w.codes_t || !a.w.scales_t || !a.w.fields) return hipErrorInvalidValue;
    if (!a.hl || !a.Xf || !a.xa || !a.xs) return hipErrorInvalidValue;
    if (a.nsplit < 1 || (a.nsplit > 1 && !a.part)) return hipErrorInvalidValue;
    if (a.w.k > 0 && (!a.tmp_k || !a.w.U)) return hipErrorInvalidValue;
    if (a.w.n_pts == 217) return launch_hexmm_tb<217>(a, st);
    if (a.w.n_pts == 127) return launch_hexmm_tb<127>(a, st);
    return launch_hexmm_tb<0>(a, st);
}

hipError_t launch_batch_prep(const BatchPrep& p, hipStream_t st) {
    if (p.M <= 0 || p.cols <= 0 || p.cols % 64 || p.ldx < p.cols || !p.X || !p.xa || !p.xs || !p.xn)
        return hipErrorInvalidValue;
    for (int g = 0; g < kMaxSeg; g++)
        if (p.k[g] < 0 || p.k[g] > kMaxRank || (p.k[g] > 0 && (!p.Vt[g] || !p.S[g] || !p.tmp[g])))
            return hipErrorInvalidValue;
    // inputs of at most kPrep2MaxCols columns, ranks <= 2, rows 16-byte
    // aligned: the four-pass kernel (row in LDS)
    bool fast = p.cols <= kPrep2MaxCols && p.ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(p.X) & 15) == 0 &&
                (reinterpret_cast<uintptr_t>(p.xn) & 15) == 0 && (!p.norm_w || (reinterpret_cast<uintptr_t>(p.norm_w) & 15) == 0);
    for (int g = 0; g < kMaxSeg; g++) fast = fast && p.k[g] <= 2 && (p.k[g] == 0 || (reinterpret_cast<uintptr_t>(p.Vt[g]) & 7) == 0);
    if (fast) {
        const size_t lds = (size_t)p.cols * 4;
        static size_t attr = 0;
        if (lds > attr) {
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&batch_prep2_kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
            attr = lds;
        }
        hipLaunchKernelGGL(batch_prep2_kernel, dim3(((p.M + 15) / 16) * 16), dim3(512), lds, st, p);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(batch_prep_kernel, dim3(((p.M + 15) / 16) * 16), dim3(256), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_embed_rows(const uint16_t* embed, const int* tokens, int M, float* X, int hidden, hipStream_t st) {
    if (M <= 0) return hipSuccess;
    hipLaunchKernelGGL(embed_rows_kernel, dim3((hidden + 255) / 256, M), dim3(256), 0, st, embed, tokens, X, hidden);
    return hipGetLastError();
}

hipError_t launch_hexmm_xprep(const uint16_t* X, int M, int cols, uint4* xa, float* xs, hipStream_t st) {
    if (M <= 0 || cols <= 0 || cols % 64 || !X || !xa || !xs) return hipErrorInvalidValue;
    if (cols <= 16384 && (reinterpret_cast<uintptr_t>(X) & 15) == 0)
        hipLaunchKernelGGL(hexmm_xprep2_kernel, dim3(((M + 15) / 16) * 16), dim3(512), 0, st, X, M, cols, xa, xs);
    else
        hipLaunchKernelGGL(hexmm_xprep_kernel, dim3(((M + 15) / 16) * 16), dim3(256), 0, st, X, M, cols, xa, xs);
    return hipGetLastError();
}

hipError_t launch_hexmm(const MatmulArgs& a, hipStream_t st) {
    if (a.hl) return hipErrorInvalidValue;
    if (a.M <= 0 || a.cols <= 0 || a.cols % 64 || !a.w.codes_t || !a.w.scales_t || !a.w.fields) return hipErrorInvalidValue;
    if (a.nsplit < 1 || (a.nsplit > 1 && !a.part)) return hipErrorInvalidValue;
    if (a.w.k > 0 && (!a.tmp_k || !a.w.U)) return hipErrorInvalidValue;
    if (!a.prepped) {
        const hipError_t e = launch_hexmm_xprep(a.X, a.M, a.cols, a.xa, a.xs, st);
        if (e != hipSuccess) return e;
    }
    if (a.w.n_pts == 217) return launch_hexmm_tb<217>(a, st);
    if (a.w.n_pts == 127) return launch_hexmm_tb<127>(a, st);
    return launch_hexmm_tb<0>(a, st);
}

hipError_t launch_lowrank_batched(const uint16_t* X, const uint16_t* Vt, const float* S, float* tmp, int M, int k,
                                  int cols, hipStream_t st) {
    if (k <= 0) return hipSuccess;
    hipLaunchKernelGGL(lowrank_batched_kernel, dim3(M, k), dim3(256), 0, st, X, Vt, S, tmp, k, cols);
    return hipGetLastError();
}

hipError_t launch_lowrank(const float* x, const uint16_t* Vt, const float* S, float* tmp_k, int k, int cols,
                          hipStream_t st) {
    if (k <= 0) return hipSuccess;
    hipLaunchKernelGGL(lowrank_kernel, dim3(k), dim3(256), 0, st, x, Vt, S, tmp_k, cols);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* w, float* out, int dim, float eps, hipStream_t st) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, st, x, w, out, dim, eps);
    return hipGetLastError();
}

hipError_t launch_vec_add(float* y, const float* a, const float* b, int dim, hipStream_t st) {
    if (dim <= 0) return hipSuccess;
    hipLaunchKernelGGL(vec_add_kernel, dim3((dim + 255) / 256), dim3(256), 0, st, y, a, b, dim);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float* g, const float* u, float* out, int dim, hipStream_t st) {
    if (dim <= 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_kernel, dim3((dim + 255) / 256), dim3(256), 0, st, g, u, out, dim);
    return hipGetLastError();
}

hipError_t launch_rope_kv_rows(float* q, const float* k, const float* v, const RopeKV& r, int M, hipStream_t st) {
    if (M <= 0 || !r.cs || r.pos_dev || r.pos < 0 || r.pos + M > r.max_seq) return hipErrorInvalidValue;
    CsInline csi;
    const int half = r.hd / 2;
    int n = r.n_heads * half;
    if (r.n_kv * r.hd > n) n = r.n_kv * r.hd;
    hipLaunchKernelGGL(rope_kv_kernel, dim3((n + 255) / 256, M), dim3(256), 0, st, q, k, v, r, csi, 0);
    return hipGetLastError();
}

hipError_t launch_rope_kv(float* q, const float* k, const float* v, const RopeKV& r, const float2* cs_inline,
                          hipStream_t st) {
    CsInline csi;
    const int half = r.hd / 2;
    if (cs_inline) {
        if (half > 128) return hipErrorInvalidValue;
        for (int i = 0; i < half; i++) csi.v[i] = cs_inline[i];
    }
    int n = r.n_heads * half;
    if (r.n_kv * r.hd > n) n = r.n_kv * r.hd;
    hipLaunchKernelGGL(rope_kv_kernel, dim3((n + 255) / 256), dim3(256), 0, st, q, k, v, r, csi, cs_inline ? 1 : 0);
    return hipGetLastError();
}

// Mergers of the one-token matrix-core attention: 8 when all `blocks`
// blocks (one 512-thread block fits on a CU with room to spare) are
// resident at once on this device, else 1 (the last split's block)
static int attn_mergers(int blocks) {
    const int ncu = device_cu_count();
    return ncu > 0 && blocks <= ncu ? 8 : 1;
}

hipError_t launch_rope_attention(const AttnArgs& a, const float* k, const float* v, int interleaved,
                                 const float2* cs, hipStream_t st) {
    const int G = a.n_kv > 0 ? a.n_heads / a.n_kv : 0;
    if (a.pos_dev || !a.ws || (a.max_splits > 1 && !a.epoch && !a.dep) || !(G == 1 || G == 2 || G == 4) ||
        !(a.hd == 64 || a.hd == 128) ||
        !(a.chunk == 64 || a.chunk == 128 || a.chunk == 256) || a.max_splits > kAttnDecSplits)
        return hipErrorNotSupported;
    AttnRope r{};
    r.k = k;
    r.v = v;
    r.interleaved = interleaved;
    for (int i = 0; i < a.hd / 2; i++) r.cs[i] = cs[i];
    const dim3 grid(a.n_kv, a.max_splits);
    AttnArgs b = a;
    b.mergers = attn_mergers(a.n_kv * a.max_splits);
#define GSD_ATTN_RI(HD, GG, IL)                                                                                 \
    switch (a.chunk) {                                                                                          \
        case 64: hipLaunchKernelGGL((attn_rope_kernel<HD, GG, 8, IL>), grid, dim3(512), 0, st, b, r); break;   \
        case 128: hipLaunchKernelGGL((attn_rope_kernel<HD, GG, 16, IL>), grid, dim3(512), 0, st, b, r); break; \
        default: hipLaunchKernelGGL((attn_rope_kernel<HD, GG, 32, IL>), grid, dim3(512), 0, st, b, r); break;  \
    }
#define GSD_ATTN_R(HD, GG) \
    if (interleaved) { GSD_ATTN_RI(HD, GG, true) } else { GSD_ATTN_RI(HD, GG, false) }
    if (a.hd == 64) {
        if (G == 1) GSD_ATTN_R(64, 1) else if (G == 2) GSD_ATTN_R(64, 2) else GSD_ATTN_R(64, 4)
    } else {
        if (G == 1) GSD_ATTN_R(128, 1) else if (G == 2) GSD_ATTN_R(128, 2) else GSD_ATTN_R(128, 4)
    }
#undef GSD_ATTN_R
#undef GSD_ATTN_RI
    return hipGetLastError();
}

size_t attention_ws_bytes(int n_kv, int max_splits, int group, int hd) {
    return (size_t)n_kv * max_splits * group * (2 + hd) * 8;
}

size_t attention_ws_bytes_upto(int n_kv, int group, int hd, int max_ctx) {
    int splits = 1;
    for (int n = 1; n <= max_ctx; n++) {
        const int c = attention_chunk(n, n_kv), s = (n + c - 1) / c;
        if (s > splits) splits = s;
    }
    return attention_ws_bytes(n_kv, splits, group, hd);
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
    // the merging block holds every split's (max, sum) in its 256-entry
    // score buffer
    if (a.max_splits < 1 || a.max_splits > 256 || a.chunk > 256 || !a.ws ||
        (a.max_splits > 1 && !a.counters && !a.epoch && !a.dep))
        return hipErrorInvalidValue;
    // the device epoch advances once every KV head's last split has merged:
    // the launch's split count must be the host's (a device position lets
    // blocks past the context leave early)
    if (a.dep && (a.pos_dev || a.epoch || a.counters)) return hipErrorInvalidValue;
    const int G = a.n_heads / a.n_kv;
    // one token, G <= 4, head dim 64 / 128: the matrix-core kernel
    if ((G == 1 || G == 2 || G == 4) && (a.hd == 64 || a.hd == 128) &&
        (a.chunk == 64 || a.chunk == 128 || a.chunk == 256) && a.max_splits <= kAttnDecSplits) {
        const dim3 grid(a.n_kv, a.max_splits);
        AttnArgs b = a;
        b.mergers = attn_mergers(a.n_kv * a.max_splits);
#define GSD_ATTN_P(HD, GG)                                                                            \
    switch (a.chunk) {                                                                                \
        case 64: hipLaunchKernelGGL((attn_dec_kernel<HD, GG, 8>), grid, dim3(512), 0, st, b); break;   \
        case 128: hipLaunchKernelGGL((attn_dec_kernel<HD, GG, 16>), grid, dim3(512), 0, st, b); break; \
        default: hipLaunchKernelGGL((attn_dec_kernel<HD, GG, 32>), grid, dim3(512), 0, st, b); break;  \
    }
#define GSD_ATTN_D(HD, GG) GSD_ATTN_P(HD, GG)
        if (a.hd == 64) {
            if (G == 1) GSD_ATTN_D(64, 1) else if (G == 2) GSD_ATTN_D(64, 2) else GSD_ATTN_D(64, 4)
        } else {
            if (G == 1) GSD_ATTN_D(128, 1) else if (G == 2) GSD_ATTN_D(128, 2) else GSD_ATTN_D(128, 4)
        }
#undef GSD_ATTN_D
#undef GSD_ATTN_P
        return hipGetLastError();
    }
    const dim3 grid(a.n_kv, a.max_splits);
    // 16 waves for up to 4 query heads per KV head (8 would not fit the
    // registers of 16), else 4
#define GSD_ATTN_L(HD, GG) \
    hipLaunchKernelGGL((attn_kernel<HD, GG, GG <= 4 ? 16 : 4>), grid, dim3(GG <= 4 ? 1024 : 256), 0, st, a);
#define GSD_ATTN_G(HD)                                          \
    switch (G) {                                                \
        case 1: GSD_ATTN_L(HD, 1) break;                        \
        case 2: GSD_ATTN_L(HD, 2) break;                        \
        case 4: GSD_ATTN_L(HD, 4) break;                        \
        case 8: GSD_ATTN_L(HD, 8) break;                        \
        default: return hipErrorInvalidValue;                   \
    }
    switch (a.hd) {
        case 64: GSD_ATTN_G(64) break;
        case 128: GSD_ATTN_G(128) break;
        case 256: GSD_ATTN_G(256) break;
        default: return hipErrorInvalidValue;
    }
#undef GSD_ATTN_G
#undef GSD_ATTN_L
    return hipGetLastError();
}

hipError_t launch_prefill_attention(const PrefillAttn& a, hipStream_t st) {
    if (a.M <= 0) return hipSuccess;
    if (!a.q || !a.k_cache || !a.v_cache || !a.out || a.n_kv <= 0 || a.n_heads % a.n_kv || a.p0 < 0 || a.layer < 0 ||
        a.p0 + a.M > a.max_seq)
        return hipErrorInvalidValue;
    const int G = a.n_heads / a.n_kv;
    if (G != 1 && G != 2 && G != 4 && G != 8) return hipErrorInvalidValue;
    PrefillAttn b = a;
    b.log2g = G == 1 ? 0 : (G == 2 ? 1 : (G == 4 ? 2 : 3));
    const int T = 64 / G;
    const dim3 grid((a.M + T - 1) / T, a.n_kv);
    switch (a.hd) {
        case 64: hipLaunchKernelGGL((attn_prefill_kernel<64>), grid, dim3(256), 0, st, b); break;
        case 128: hipLaunchKernelGGL((attn_prefill_kernel<128>), grid, dim3(256), 0, st, b); break;
        case 256: hipLaunchKernelGGL((attn_prefill_kernel<256>), grid, dim3(256), 0, st, b); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_embed(const uint16_t* embed, const int* token_dev, float* x, int hidden,
                        unsigned long long* clear, int nclear, unsigned* epoch, hipStream_t st) {
    const int n = hidden > nclear ? hidden : nclear;
    hipLaunchKernelGGL(embed_kernel, dim3((n + 255) / 256), dim3(256), 0, st, embed, token_dev, x, hidden, clear,
                       nclear, epoch);
    return hipGetLastError();
}

hipError_t launch_set_step(StepState* stt, int token, int pos, int reset_err, hipStream_t st) {
    hipLaunchKernelGGL(set_step_kernel, dim3(1), dim3(1), 0, st, stt, token, pos, reset_err);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int n, StepState* stt, int* gen_tokens, float* gen_margins,
                         int advance, hipStream_t st, unsigned long long* words, unsigned* ctr) {
    if (words && ctr)
        hipLaunchKernelGGL(argmax_blocks_kernel, dim3(kArgBlocks), dim3(256), 0, st, logits, n, stt, gen_tokens,
                           gen_margins, advance, words, ctr);
    else
        hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, st, logits, n, stt, gen_tokens, gen_margins, advance);
    return hipGetLastError();
}

hipError_t launch_fill_u32(unsigned* p, unsigned v, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, v, n);
    return hipGetLastError();
}

hipError_t launch_unpack(const uint8_t* codes, int64_t n, int radius, int32_t* idx, int8_t* r01, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, codes, n, radius, idx, r01);
    return hipGetLastError();
}

// Codes of a tiled tensor back in file order (u8 [rows][cols / 2]), decoded
// with the tile helpers the matvec kernels use: one wave per tile.
__global__ void __launch_bounds__(64) tile_codes_kernel(const uint4* codes_t, int rows, int cols, int n_pts,
                                                        uint8_t* out) {
    const int lane = threadIdx.x;
    const int nc = (cols + 127) >> 7, half = cols >> 1;
    const int rb = (int)blockIdx.x / nc, c = (int)blockIdx.x % nc;
    const bool b7 = n_pts <= 128;
    const unsigned char* tile = reinterpret_cast<const unsigned char*>(codes_t) + ((size_t)rb * nc + c) * tile_bytes(b7);
    const uint4 q = tile_load(tile + tile_lane_off(b7, lane));
    uint32_t w[4] = {q.x, q.y, q.z, q.w};
    if (b7) align7(w, (uint32_t)(lane & 1) * 16u);
    const int row = rb * 16 + (lane & 15);
    if (row >= rows) return;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int p = 64 * c + (j < 8 ? 8 * (lane >> 4) + j : 32 + 8 * (lane >> 4) + (j - 8));
        if (p < half) out[(size_t)row * half + p] = (uint8_t)code_of(w, j, b7);
    }
}

hipError_t launch_tile_codes(const HexSeg& s, int cols, uint8_t* out, hipStream_t st) {
    if (!s.codes_t || !out || s.rows <= 0 || cols <= 0 || cols % 64) return hipErrorInvalidValue;
    const size_t tiles = (size_t)((s.rows + 15) / 16) * ((cols + 127) / 128);
    hipLaunchKernelGGL(tile_codes_kernel, dim3((unsigned)tiles), dim3(64), 0, st, s.codes_t, s.rows, cols, s.n_pts, out);
    return hipGetLastError();
}

hipError_t launch_copy(const void* src, void* dst, size_t nbytes, hipStream_t st) {
    if (nbytes % 16) return hipErrorInvalidValue;
    const size_t n = nbytes / 16;
    if (n == 0) return hipSuccess;
    size_t grid = (n + 255) / 256;
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(copy_kernel, dim3((unsigned)grid), dim3(256), 0, st, reinterpret_cast<const uint4*>(src),
                       reinterpret_cast<uint4*>(dst), n);
    return hipGetLastError();
}

int device_cu_count() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return n;
}

}  // namespace gsd
