/*
 * gsdref.c -- CPU oracle for the GSD-LQ batch-1 decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP engine is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load the library built from it; the product library
 * (libgsdhip.so) never links, loads or calls it.
 *
 * It restates, function by function, the arithmetic of the reference CPU
 * engine gsd_lq_v2/gsd_lq_cpu_engine.c (cited per function below):
 *   - the same loop order and sequential fp32 accumulation,
 *   - IEEE binary16 conversions with round-to-nearest-even (the reference
 *     uses a _Float16 cast, gsd_lq_cpu_engine.c:27-40; here the conversion is
 *     written out in integer arithmetic so that gcc can build it too),
 *   - 1/sqrtf, expf, powf, cosf, sinf from the C library, called per element
 *     exactly where the reference calls them.
 * One deliberate difference: the attention scores buffer is on the heap, so
 * contexts longer than the reference's fixed float scores[2048]
 * (gsd_lq_cpu_engine.c:292) are well defined.  For pos < 2048 the arithmetic
 * is identical.
 *
 * The exported gsd_cpu_* names and argument orders are the reference's
 * interface (gsd_lq_v2/gsd_lq_cpu_runtime.py:91-108), so one ctypes driver can
 * run either this oracle or the reference library built from source.
 *
 * Build flags follow the reference runtime (gsd_lq_cpu_runtime.py:45-55):
 *   clang -O3 -shared -fPIC -fopenmp   (no -march: scalar SSE2, no FMA).
 *
 * Pinning: every function here is checked in tests/ against golden vectors
 * written by the reference engine itself (tests/golden/), against the
 * reference library directly when it is built (oracle/_ref), and against
 * closed forms / float64 brute force.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------- */
/* IEEE 754 binary16 <-> binary32 (gsd_lq_cpu_engine.c:27-40 semantics)    */
/* ---------------------------------------------------------------------- */

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Exact widening: every binary16 value (incl. subnormals, inf, NaN payload)
 * is representable in binary32. */
static inline float h2f(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1Fu) {                         /* inf / NaN */
        return bits_f32(sign | 0x7F800000u | (m << 13));
    }
    if (e == 0) {
        if (m == 0) return bits_f32(sign);    /* signed zero */
        /* subnormal: value = m * 2^-24, exact in binary32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* Narrowing with round-to-nearest-even, gradual underflow, overflow to inf.
 * NaN keeps its sign and top payload bits and is made quiet (what both the
 * x86 F16C instruction and compiler-rt's __truncsfhf2 produce). */
static inline uint16_t f2h(float f)
{
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) {
        if (a == 0x7F800000u) return sign | 0x7C00u;
        return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
    }
    /* largest value that rounds to a finite half is 65519.99...; from
     * 65520 (0x477FF000) upward the result is inf. */
    if (a >= 0x477FF000u) return sign | 0x7C00u;
    if (a < 0x38800000u) {
        /* result is subnormal or zero: quantum 2^-24 */
        if (a < 0x33000000u) return sign;     /* < 2^-25: rounds to zero */
        uint32_t e = a >> 23;                 /* biased exponent, 102..112 */
        uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;            /* 14..24 */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    /* normal range: rebias exponent, round 13 dropped mantissa bits */
    uint32_t r = a - 0x38000000u;             /* exponent 127 -> 15 */
    uint32_t q = r >> 13;
    uint32_t rem = r & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

void gsdref_f16_to_f32(const uint16_t* h, float* out, long n)
{
    for (long i = 0; i < n; i++) out[i] = h2f(h[i]);
}

void gsdref_f32_to_f16(const float* f, uint16_t* out, long n)
{
    for (long i = 0; i < n; i++) out[i] = f2h(f[i]);
}

/* ---------------------------------------------------------------------- */
/* 1. RMSNorm  (gsd_lq_cpu_engine.c:66-82)                                 */
/* ---------------------------------------------------------------------- */
void gsd_cpu_rmsnorm(const float* x, const float* weight, float* out, int dim, float eps)
{
    float ss = 0.0f;
    int i;
    for (i = 0; i < dim; i++) ss += x[i] * x[i];
    float inv = 1.0f / sqrtf((ss / (float)dim) + eps);
    for (i = 0; i < dim; i++) out[i] = x[i] * inv * weight[i];
}

/* 2. y = a + b  (gsd_lq_cpu_engine.c:84-94) */
void gsd_cpu_vec_add(float* y, const float* a, const float* b, int dim)
{
    for (int i = 0; i < dim; i++) y[i] = a[i] + b[i];
}

/* 3. out = silu(gate) * up, no clamp  (gsd_lq_cpu_engine.c:96-108) */
void gsd_cpu_swiglu(const float* gate, const float* up, float* out, int dim)
{
    for (int i = 0; i < dim; i++) {
        float g = gate[i];
        float s = g / (1.0f + expf(-g));
        out[i] = s * up[i];
    }
}

/* 4. tmp_k[j] = (sum_c x[c] * Vt[j,c]) * S[j]  (gsd_lq_cpu_engine.c:110-127) */
void gsd_cpu_lowrank_proj(const float* x, const uint16_t* Vt, const float* S,
                          float* tmp_k, int k_dim, int cols)
{
    for (int j = 0; j < k_dim; j++) {
        const uint16_t* vrow = Vt + (size_t)j * (size_t)cols;
        float d = 0.0f;
        for (int c = 0; c < cols; c++) d += x[c] * h2f(vrow[c]);
        tmp_k[j] = d * S[j];
    }
}

/* 5. Fused hex2d matvec  (gsd_lq_cpu_engine.c:129-183)
 *    acc = sum_p (T[code].x * x[2p] + T[code].y * x[2p+1]) * scale[blk]
 *        + sum_kinks delta * x[col]
 *        + sum_j U[r,j] * tmp_k[j]                       (in that order) */
void gsd_cpu_hex2d_matvec(const float* x, const uint8_t* codes, const uint16_t* scales,
                          const float* xy_table, const uint16_t* U, const float* tmp_k,
                          const uint32_t* kink_row_ptr, const uint16_t* kink_cols,
                          const float* kink_deltas, float* y,
                          int rows, int cols, int k_dim, int n_pts)
{
    (void)n_pts;   /* unused by the reference CPU engine as well */
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const size_t first = (size_t)r * (size_t)cols;   /* flat weight index */
        const uint8_t* crow = codes + (first >> 1);
        const uint16_t* srow = scales + (first >> 6);
        const int npairs = cols >> 1;
        float acc = 0.0f;
        for (int p = 0; p < npairs; p++) {
            float s = h2f(srow[p >> 5]);
            unsigned c = crow[p];
            float tx = xy_table[2u * c];
            float ty = xy_table[2u * c + 1u];
            acc += (tx * x[2 * p] + ty * x[2 * p + 1]) * s;
        }
        for (uint32_t i = kink_row_ptr[r]; i < kink_row_ptr[r + 1]; i++)
            acc += kink_deltas[i] * x[kink_cols[i]];
        if (k_dim > 0) {
            const uint16_t* urow = U + (size_t)r * (size_t)k_dim;
            for (int j = 0; j < k_dim; j++) acc += h2f(urow[j]) * tmp_k[j];
        }
        y[r] = acc;
    }
}

/* ---------------------------------------------------------------------- */
/* 6. RoPE on q (in place) and k, append k', v to the fp16 cache           */
/*    (gsd_lq_cpu_engine.c:185-262).  Cache layout [layer][pos][kvh][d].   */
/* ---------------------------------------------------------------------- */
void gsd_cpu_rope_and_store_kv(float* q, const float* k, const float* v,
                               uint16_t* k_cache, uint16_t* v_cache,
                               int layer_idx, int pos, int n_heads, int n_kv_heads,
                               int head_dim, int max_seq_len, float rope_theta,
                               int interleaved)
{
    const int half = head_dim / 2;
    const size_t row = (size_t)n_kv_heads * (size_t)head_dim;
    const size_t base = (size_t)layer_idx * (size_t)max_seq_len * row + (size_t)pos * row;

    for (size_t i = 0; i < row; i++) v_cache[base + i] = f2h(v[i]);

    for (int h = 0; h < n_heads; h++) {
        float* qh = q + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            float freq = 1.0f / powf(rope_theta, (float)(2 * i) / (float)head_dim);
            float ang = (float)pos * freq;
            float c = cosf(ang), s = sinf(ang);
            int i0 = interleaved ? 2 * i : i;
            int i1 = interleaved ? 2 * i + 1 : i + half;
            float a = qh[i0], b = qh[i1];
            qh[i0] = a * c - b * s;
            qh[i1] = a * s + b * c;
        }
    }
    for (int h = 0; h < n_kv_heads; h++) {
        const float* kh = k + (size_t)h * head_dim;
        uint16_t* dst = k_cache + base + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            float freq = 1.0f / powf(rope_theta, (float)(2 * i) / (float)head_dim);
            float ang = (float)pos * freq;
            float c = cosf(ang), s = sinf(ang);
            int i0 = interleaved ? 2 * i : i;
            int i1 = interleaved ? 2 * i + 1 : i + half;
            float a = kh[i0], b = kh[i1];
            dst[i0] = f2h(a * c - b * s);
            dst[i1] = f2h(a * s + b * c);
        }
    }
}

/* ---------------------------------------------------------------------- */
/* 7. GQA decode attention over cached positions 0..pos                    */
/*    (gsd_lq_cpu_engine.c:264-330): scores, max, exp, sum, scale by 1/sum, */
/*    then out = sum_t p_t * V_t, all sequential in t.                      */
/* ---------------------------------------------------------------------- */
void gsd_cpu_gqa_attention(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                           float* attn_out, int layer_idx, int pos, int n_heads,
                           int n_kv_heads, int head_dim, int max_seq_len, float sm_scale)
{
    const int group = n_heads / n_kv_heads;
    const size_t row = (size_t)n_kv_heads * (size_t)head_dim;
    const size_t lbase = (size_t)layer_idx * (size_t)max_seq_len * row;
    const int n = pos + 1;

    #pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; h++) {
        const int kvh = h / group;
        const float* qh = q + (size_t)h * head_dim;
        float* oh = attn_out + (size_t)h * head_dim;
        float* p = (float*)malloc((size_t)n * sizeof(float));
        float mx = -1e30f;
        for (int t = 0; t < n; t++) {
            const uint16_t* kt = k_cache + lbase + (size_t)t * row + (size_t)kvh * head_dim;
            float d = 0.0f;
            for (int i = 0; i < head_dim; i++) d += qh[i] * h2f(kt[i]);
            float s = d * sm_scale;
            p[t] = s;
            if (s > mx) mx = s;
        }
        float sum = 0.0f;
        for (int t = 0; t < n; t++) {
            float e = expf(p[t] - mx);
            p[t] = e;
            sum += e;
        }
        float inv = 1.0f / sum;
        for (int t = 0; t < n; t++) p[t] *= inv;
        for (int i = 0; i < head_dim; i++) oh[i] = 0.0f;
        for (int t = 0; t < n; t++) {
            const float w = p[t];
            const uint16_t* vt = v_cache + lbase + (size_t)t * row + (size_t)kvh * head_dim;
            for (int i = 0; i < head_dim; i++) oh[i] += w * h2f(vt[i]);
        }
        free(p);
    }
}

/* ---------------------------------------------------------------------- */
/* Helpers used only by tests: codebook and exhaustive index decoding.      */
/* ---------------------------------------------------------------------- */

/* A2 hexagon of radius R, r0 outer, r1 inner, |r0+r1| <= R; point =
 * (r0 + r1/2, r1*sqrt(3)/2) evaluated in double, stored as float
 * (gsd_lq_cpu_runtime.py:111-118, run_gpu_native_chat.py:26-33).
 * Writes n_pts (x,y) pairs to xy and the integer fields to r01 (2 per
 * point); returns n_pts. */
int gsdref_codebook(int radius, float* xy, int8_t* r01)
{
    const double s32 = sqrt(3.0) / 2.0;
    int n = 0;
    for (int a = -radius; a <= radius; a++)
        for (int b = -radius; b <= radius; b++) {
            if (abs(a + b) > radius) continue;
            if (xy) { xy[2 * n] = (float)((double)a + 0.5 * (double)b); xy[2 * n + 1] = (float)((double)b * s32); }
            if (r01) { r01[2 * n] = (int8_t)a; r01[2 * n + 1] = (int8_t)b; }
            n++;
        }
    return n;
}

/* Dense dequantized row-major matrix W[r,c] = T[code].{x|y} * scale, plus the
 * kinks (added as separate terms) -- the brute-force view of the format. */
void gsdref_dequant(const uint8_t* codes, const uint16_t* scales, const float* xy_table,
                    const uint32_t* kink_row_ptr, const uint16_t* kink_cols,
                    const float* kink_deltas, double* W, int rows, int cols)
{
    for (int r = 0; r < rows; r++) {
        for (int c = 0; c < cols; c++) {
            size_t i = (size_t)r * cols + c;
            unsigned code = codes[i >> 1];
            double t = xy_table[2u * code + (unsigned)(i & 1u)];
            W[i] = t * (double)h2f(scales[i >> 6]);
        }
        for (uint32_t k = kink_row_ptr[r]; k < kink_row_ptr[r + 1]; k++)
            W[(size_t)r * cols + kink_cols[k]] += (double)kink_deltas[k];
    }
}
