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
//   * prologue fusions: RMSNorm of the input and the rank-k projection
//     tmp_k = S * (Vt x) are recomputed per block from the register slice;
//   * epilogue fusions: kinks and the U tmp_k term, then store / residual add /
//     SwiGLU of paired gate-up rows.
#include "gsd_internal.h"

namespace gsd {
namespace {

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sum over the block; every thread gets the total.  lds: >= 16 floats.
__device__ float block_sum(float v, float* lds) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) lds[wid] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < nw; w++) t += lds[w];
    return t;
}

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

template <int SPT, int MAXT, int RB>
__global__ void __launch_bounds__(MAXT) hexmv_kernel(const HexArgs a) {
    __shared__ float2 tbl[kMaxSeg][kTableSlots];
    __shared__ float red[MAXT / 64][RB];
    __shared__ float fin[RB];
    __shared__ float tkl[kMaxSeg][kMaxRank];
    __shared__ float scratch[16];
    __shared__ float s_inv;

    const int tid = threadIdx.x, NT = blockDim.x, lane = tid & 63, wid = tid >> 6;
    const int NW = NT >> 6;
    const int S = a.cols >> 5;
    const int nsb = a.cols >> 6;
    const size_t rowbytes = (size_t)(a.cols >> 1);

    for (int g = 0; g < a.nseg; g++) {
        const float2* tg = reinterpret_cast<const float2*>(a.seg[g].table);
        for (int i = tid; i < kTableSlots; i += NT) tbl[g][i] = i < a.seg[g].n_pts ? tg[i] : make_float2(0.f, 0.f);
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

    // fused rank-k projection (gsd_lq_cpu_engine.c:110-127)
    for (int g = 0; g < a.nseg; g++) {
        const HexSeg& sg = a.seg[g];
        if (sg.k <= 0) continue;
        if (sg.tmp_k) {
            if (tid < sg.k) tkl[g][tid] = sg.tmp_k[tid];
            continue;
        }
        for (int jj = 0; jj < sg.k; jj++) {
            float p = 0.f;
#pragma unroll
            for (int j = 0; j < SPT; j++) {
                const int s = tid + j * NT;
                if (s < S) {
                    const uint4* vp = reinterpret_cast<const uint4*>(sg.Vt + (size_t)jj * a.cols + (size_t)s * 32);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const uint4 v = vp[q];
                        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            p = fmaf(xr[j][8 * q + 2 * e], h2f((uint16_t)(w[e] & 0xFFFFu)), p);
                            p = fmaf(xr[j][8 * q + 2 * e + 1], h2f((uint16_t)(w[e] >> 16)), p);
                        }
                    }
                }
            }
            p = block_sum(p, scratch);
            if (tid == 0) tkl[g][jj] = p * sg.S[jj];
        }
    }
    __syncthreads();

    const bool paired = a.epilogue == kEpiSwiGLU;
    for (int b = blockIdx.x; b < a.nbatch; b += gridDim.x) {
        // rows of this batch: paired -> RB/2 rows of seg0 and the same of seg1
        int gsel = 0, r0 = 0;
        if (paired) {
            r0 = b * (RB / 2);
        } else {
            while (gsel + 1 < a.nseg && b >= a.seg[gsel + 1].batch0) gsel++;
            r0 = (b - a.seg[gsel].batch0) * RB;
        }
        float acc[RB];
#pragma unroll
        for (int rr = 0; rr < RB; rr++) acc[rr] = 0.f;

#pragma unroll
        for (int j = 0; j < SPT; j++) {
            const int s = tid + j * NT;
            if (s >= S) continue;
            uint4 cw[RB];
            uint16_t sc[RB];
#pragma unroll
            for (int rr = 0; rr < RB; rr++) {
                const int g = paired ? (rr >= RB / 2) : gsel;
                const int row = paired ? r0 + (rr % (RB / 2)) : r0 + rr;
                if (row < a.seg[g].rows) {
                    cw[rr] = *reinterpret_cast<const uint4*>(a.seg[g].codes + (size_t)row * rowbytes + (size_t)s * 16);
                    sc[rr] = a.seg[g].scales[(size_t)row * nsb + (s >> 1)];
                } else {
                    cw[rr] = make_uint4(0, 0, 0, 0);
                    sc[rr] = 0;
                }
            }
#pragma unroll
            for (int rr = 0; rr < RB; rr++) {
                const int g = paired ? (rr >= RB / 2) : gsel;
                acc[rr] = fmaf(dot16(cw[rr], tbl[g], xr[j]), h2f(sc[rr]), acc[rr]);
            }
        }
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            const float v = wave_sum(acc[rr]);
            if (lane == 0) red[wid][rr] = v;
        }
        __syncthreads();
        if (tid < RB) {
            const int rr = tid;
            const int g = paired ? (rr >= RB / 2) : gsel;
            const int row = paired ? r0 + (rr % (RB / 2)) : r0 + rr;
            const HexSeg& sg = a.seg[g];
            float t = 0.f;
            for (int w = 0; w < NW; w++) t += red[w][rr];
            if (row < sg.rows) {
                if (sg.row_ptr) {
                    const uint32_t e = sg.row_ptr[row + 1];
                    for (uint32_t i = sg.row_ptr[row]; i < e; i++) {
                        const int c = sg.kcols[i];
                        const float xc = a.norm_w ? (a.x[c] * s_inv) * a.norm_w[c] : a.x[c];
                        t += sg.kdel[i] * xc;
                    }
                }
                for (int jj = 0; jj < sg.k; jj++) t += h2f(sg.U[(size_t)row * sg.k + jj]) * tkl[g][jj];
                if (a.epilogue == kEpiStore) sg.out[row] = t;
                else if (a.epilogue == kEpiResidual) a.resid[row] = a.resid[row] + t;
            }
            fin[rr] = t;
        }
        if (paired) {
            __syncthreads();
            if (tid < RB / 2) {
                const int row = r0 + tid;
                if (row < a.seg[0].rows) {
                    const float gt = fin[tid], up = fin[tid + RB / 2];
                    a.seg[0].out[row] = (gt / (1.0f + expf(-gt))) * up;
                }
            }
        }
        __syncthreads();
    }
}

template <int SPT, int MAXT>
hipError_t launch_hexmv_t(const HexArgs& a, hipStream_t st, int nt) {
    constexpr int RB = 8;
    HexArgs b = a;
    // batches: per segment ceil(rows/RB), or ceil(rows/(RB/2)) paired
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
    const int grid = b.nbatch < 4096 ? b.nbatch : 4096;
    hipLaunchKernelGGL((hexmv_kernel<SPT, MAXT, RB>), dim3(grid), dim3(nt), 0, st, b);
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
    const int pos = r.pos_dev ? *r.pos_dev : r.pos;
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
// grid = (n_kv, max_splits); a block handles one KV head, all `group` query
// heads that share it (K/V read once per group, not once per query head),
// and `chunk` (<= 256) positions.  The last block of a KV head to finish
// merges the per-split (max, sum, o) partials.
// ------------------------------------------------------------------------
template <int HD>
__global__ void __launch_bounds__(256) attn_kernel(const AttnArgs a) {
    constexpr int DG = HD / 8;          // 8-dim groups (16-byte loads)
    constexpr int PL = 256 / DG;        // position lanes in phase C
    constexpr int MAXG = 8;
    __shared__ float qs[MAXG][HD];
    __shared__ float sc[MAXG][256];
    __shared__ float part[4][MAXG][HD];
    __shared__ float mred[4][MAXG];
    __shared__ float ml[2][MAXG];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int pos = a.pos_dev ? *a.pos_dev : a.pos;
    const int n = pos + 1;
    const int nsplit = (n + a.chunk - 1) / a.chunk;
    const int split = blockIdx.y;
    if (split >= nsplit) return;
    const int kvh = blockIdx.x;
    const int G = a.n_heads / a.n_kv;
    const int t0 = split * a.chunk;
    const int t1 = min(n, t0 + a.chunk);
    const size_t rowstride = (size_t)a.n_kv * HD;
    const size_t lbase = (size_t)a.layer * a.max_seq * rowstride + (size_t)kvh * HD;

    for (int i = tid; i < G * HD; i += 256) qs[i / HD][i % HD] = a.q[(size_t)(kvh * G) * HD + i];
    __syncthreads();

    // phase A: scores, one position per thread, dot in the reference order
    {
        const int t = t0 + tid;
        if (t < t1) {
            float dot[MAXG];
#pragma unroll
            for (int g = 0; g < MAXG; g++) dot[g] = 0.f;
            const uint4* kp = reinterpret_cast<const uint4*>(a.k_cache + lbase + (size_t)t * rowstride);
            for (int d8 = 0; d8 < DG; d8++) {
                const uint4 kv = kp[d8];
                const uint32_t w[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float kf = h2f((uint16_t)(w[e >> 1] >> (16 * (e & 1))));
#pragma unroll
                    for (int g = 0; g < MAXG; g++) {
                        if (g < G) {
#pragma clang fp contract(off)
                            dot[g] = dot[g] + qs[g][d8 * 8 + e] * kf;
                        }
                    }
                }
            }
#pragma unroll
            for (int g = 0; g < MAXG; g++)
                if (g < G) sc[g][tid] = dot[g] * a.sm_scale;
        }
    }
    __syncthreads();
    // phase B: per-head max and exp-sum over this chunk
    const int cn = t1 - t0;
    for (int g = 0; g < G; g++) {
        float m = tid < cn ? sc[g][tid] : -INFINITY;
        m = wave_max(m);
        if (lane == 0) mred[wid][g] = m;
    }
    __syncthreads();
    if (tid < G) ml[0][tid] = fmaxf(fmaxf(mred[0][tid], mred[1][tid]), fmaxf(mred[2][tid], mred[3][tid]));
    __syncthreads();
    for (int g = 0; g < G; g++) {
        float e = 0.f;
        if (tid < cn) {
            e = expf(sc[g][tid] - ml[0][g]);
            sc[g][tid] = e;
        }
        e = wave_sum(e);
        if (lane == 0) mred[wid][g] = e;
    }
    __syncthreads();
    if (tid < G) ml[1][tid] = (mred[0][tid] + mred[1][tid]) + (mred[2][tid] + mred[3][tid]);
    // phase C: o[g][d] = sum_t p[g][t] V_t[d]
    {
        const int dg = tid % DG, pl = tid / DG;
        float acc[MAXG][8];
#pragma unroll
        for (int g = 0; g < MAXG; g++)
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] = 0.f;
        for (int t = t0 + pl; t < t1; t += PL) {
            const uint4 vv = *reinterpret_cast<const uint4*>(a.v_cache + lbase + (size_t)t * rowstride + dg * 8);
            const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
            float vf[8];
#pragma unroll
            for (int e = 0; e < 8; e++) vf[e] = h2f((uint16_t)(w[e >> 1] >> (16 * (e & 1))));
#pragma unroll
            for (int g = 0; g < MAXG; g++) {
                if (g < G) {
                    const float p = sc[g][t - t0];
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
                }
            }
        }
        // reduce over position lanes inside the wave (lanes dg + DG*k)
#pragma unroll
        for (int o = DG; o < 64; o <<= 1)
#pragma unroll
            for (int g = 0; g < MAXG; g++)
#pragma unroll
                for (int e = 0; e < 8; e++) acc[g][e] += __shfl_xor(acc[g][e], o, 64);
        if (lane < DG) {
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int e = 0; e < 8; e++) part[wid][g][dg * 8 + e] = acc[g][e];
        }
    }
    __syncthreads();
    const int group_base = kvh * G;
    if (nsplit == 1) {
        for (int i = tid; i < G * HD; i += 256) {
            const int g = i / HD, d = i % HD;
            const float o = (part[0][g][d] + part[1][g][d]) + (part[2][g][d] + part[3][g][d]);
            a.out[(size_t)(group_base + g) * HD + d] = o * (1.0f / ml[1][g]);
        }
        return;
    }
    // write partials [kvh][split][g][2+HD]
    float* wsb = a.ws + ((size_t)kvh * a.max_splits + split) * G * (2 + HD);
    for (int i = tid; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        wsb[g * (2 + HD) + 2 + d] = (part[0][g][d] + part[1][g][d]) + (part[2][g][d] + part[3][g][d]);
    }
    if (tid < G) {
        wsb[tid * (2 + HD)] = ml[0][tid];
        wsb[tid * (2 + HD) + 1] = ml[1][tid];
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = atomicAdd(&a.counters[kvh], 1u);
        s_last = (prev == (unsigned)(nsplit - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const float* base = a.ws + (size_t)kvh * a.max_splits * G * (2 + HD);
    for (int i = tid; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        float M = -INFINITY;
        for (int sp = 0; sp < nsplit; sp++) M = fmaxf(M, __builtin_nontemporal_load(base + ((size_t)sp * G + g) * (2 + HD)));
        float L = 0.f, O = 0.f;
        for (int sp = 0; sp < nsplit; sp++) {
            const float* pp = base + ((size_t)sp * G + g) * (2 + HD);
            const float f = expf(__builtin_nontemporal_load(pp) - M);
            L = fmaf(__builtin_nontemporal_load(pp + 1), f, L);
            O = fmaf(__builtin_nontemporal_load(pp + 2 + d), f, O);
        }
        a.out[(size_t)(group_base + g) * HD + d] = O / L;
    }
    if (tid == 0) a.counters[kvh] = 0u;
}

__global__ void embed_kernel(const uint16_t* embed, const int* token, float* x, int hidden) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < hidden) x[i] = h2f(embed[(size_t)(*token) * hidden + i]);
}

// greedy argmax: nan -> -1e4, +inf -> 100, -inf -> -1e4, first index wins
__device__ __forceinline__ float clean(float v) {
    if (v != v) return -1e4f;
    if (v == INFINITY) return 100.f;
    if (v == -INFINITY) return -1e4f;
    return v;
}

__global__ void __launch_bounds__(1024) argmax_kernel(const float* logits, int n, StepState* st, int* gen_tok,
                                                      float* gen_margin, int advance) {
    __shared__ float sv1[1024], sv2[1024];
    __shared__ int si1[1024];
    const int tid = threadIdx.x;
    float v1 = -INFINITY, v2 = -INFINITY;
    int i1 = 0x7FFFFFFF;
    for (int i = tid; i < n; i += blockDim.x) {
        const float v = clean(logits[i]);
        if (v > v1) { v2 = v1; v1 = v; i1 = i; }
        else if (v > v2) v2 = v;
    }
    sv1[tid] = v1; sv2[tid] = v2; si1[tid] = i1;
    __syncthreads();
    for (int s = blockDim.x >> 1; s > 0; s >>= 1) {
        if (tid < s) {
            const float a1 = sv1[tid], a2 = sv2[tid], b1 = sv1[tid + s], b2 = sv2[tid + s];
            const int ai = si1[tid], bi = si1[tid + s];
            if (b1 > a1 || (b1 == a1 && bi < ai)) {
                sv1[tid] = b1; si1[tid] = bi; sv2[tid] = fmaxf(a1, b2);
            } else {
                sv2[tid] = fmaxf(a2, b1);
            }
        }
        __syncthreads();
    }
    if (tid == 0) {
        const int tok = si1[0];
        const float margin = sv1[0] - sv2[0];
        st->token = tok;
        if (gen_tok) {
            const int c = st->gen_count;
            gen_tok[c] = tok;
            gen_margin[c] = margin;
            st->gen_count = c + 1;
        }
        if (advance) st->pos = st->pos + 1;
        st->pad = __float_as_int(margin);
    }
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

}  // namespace

// ------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------
hipError_t launch_hexmv(const HexArgs& a, hipStream_t st) {
    const int S = a.cols >> 5;
    const int spt = (S % 128 == 0) ? 2 : 1;
    const int nt = ((S + spt - 1) / spt + 63) / 64 * 64;
    if (nt > 1024) return hipErrorInvalidValue;
    if (spt == 2) {
        if (nt <= 64) return launch_hexmv_t<2, 64>(a, st, nt);
        if (nt <= 256) return launch_hexmv_t<2, 256>(a, st, nt);
        if (nt <= 512) return launch_hexmv_t<2, 512>(a, st, nt);
        return launch_hexmv_t<2, 1024>(a, st, nt);
    }
    if (nt <= 64) return launch_hexmv_t<1, 64>(a, st, nt);
    if (nt <= 256) return launch_hexmv_t<1, 256>(a, st, nt);
    if (nt <= 512) return launch_hexmv_t<1, 512>(a, st, nt);
    return launch_hexmv_t<1, 1024>(a, st, nt);
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

size_t attention_ws_floats(int n_kv, int max_splits, int group, int hd) {
    return (size_t)n_kv * max_splits * group * (2 + hd);
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
    const dim3 grid(a.n_kv, a.max_splits);
    switch (a.hd) {
        case 64: hipLaunchKernelGGL(attn_kernel<64>, grid, dim3(256), 0, st, a); break;
        case 128: hipLaunchKernelGGL(attn_kernel<128>, grid, dim3(256), 0, st, a); break;
        case 256: hipLaunchKernelGGL(attn_kernel<256>, grid, dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_embed(const uint16_t* embed, const int* token_dev, float* x, int hidden, hipStream_t st) {
    hipLaunchKernelGGL(embed_kernel, dim3((hidden + 255) / 256), dim3(256), 0, st, embed, token_dev, x, hidden);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int n, StepState* stt, int* gen_tokens, float* gen_margins,
                         int advance, hipStream_t st) {
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

int device_cu_count() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return n;
}

}  // namespace gsd
