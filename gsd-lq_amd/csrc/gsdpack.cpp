// gsdpack.cpp -- host-side GSD-LQ encoder (packer) and synthetic weights.
//
// The reference ships no encoder: its loaders fix the .gsd2 format
// (gsd_lq_v2/run_gpu_native_chat.py:788-814, gsd_lq_cpu_runtime.py:173-199)
// but not how codes, scales, kinks and the low-rank factors are chosen.  This
// file is this project's encoder for that format:
//
//   scales : per 64-weight block, s = fp16_up(max_pairs hexnorm(a, b) / R),
//            where (a, b) are the pair's coordinates in the lattice basis
//            (1, 0), (1/2, sqrt(3)/2) and hexnorm = max(|a|, |b|, |a+b|);
//            rounding the fp16 scale up keeps every pair inside the hexagon.
//   codes  : nearest A2 lattice point of (a, b)/s among the corners of the
//            lattice cell containing it, restricted to the radius-R hexagon;
//            index = position in the codebook enumeration.
//   kinks  : optional, per row the kinks_per_row weights with the largest
//            |residual|, stored as (column, fp32 delta = residual).
//   U,S,Vt : optional rank-k factorisation of the residual E = W - W_hat by
//            subspace iteration (lr_iters rounds) and a Gram-Schmidt QR;
//            U orthonormal, S = row norms of R Q^T, Vt = normalised rows.
//
// All float work runs in a fixed order (OpenMP splits only independent rows or
// columns), so the output bytes do not depend on the thread count or machine.
//
// The synthetic generator gives reproducible ~N(0, sigma) weights from a
// counter-based hash: each value is an Irwin-Hall(12) sum of twelve 16-bit
// uniforms drawn from splitmix64(key + i), which is exact integer arithmetic,
// then one IEEE multiply and a round-to-nearest-even to bf16 (or fp16).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

inline uint32_t fbits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float bitsf(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0x1Fu) return bitsf(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        if (!m) return bitsf(sign);
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return bitsf(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t float_to_half(float f) {   // IEEE round-to-nearest-even
    uint32_t u = fbits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return a == 0x7F800000u ? (sign | 0x7C00u) : (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
    if (a >= 0x477FF000u) return sign | 0x7C00u;
    if (a < 0x38800000u) {
        if (a < 0x33000000u) return sign;
        uint32_t e = a >> 23, mant = (a & 0x7FFFFFu) | 0x800000u, sh = 126u - e;
        uint32_t q = mant >> sh, rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = a - 0x38000000u, q = r >> 13, rem = r & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return splitmix64(seed ^ splitmix64(stream + 0x632BE59BD9B4E019ull));
}

// Irwin-Hall(12) integer sum centred at zero; variance ~ 65536^2.
inline int32_t ih12(uint64_t key, int64_t i) {
    int64_t s = 0;
    for (int j = 0; j < 3; j++) {
        uint64_t h = splitmix64(key + (uint64_t)(3 * i + j));
        s += (int64_t)(h & 0xFFFF) + (int64_t)((h >> 16) & 0xFFFF) + (int64_t)((h >> 32) & 0xFFFF) + (int64_t)(h >> 48);
    }
    return (int32_t)(s - 393210);   // 12 * 32767.5
}

inline float round_bf16(float f) {
    uint32_t u = fbits(f);
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
    return bitsf(u);
}

struct Codebook {
    int R = 0, n = 0;
    std::vector<float> xy;       // n * 2
    std::vector<int> index;      // (2R+1)^2, -1 outside
    explicit Codebook(int radius) : R(radius) {
        const double s32 = std::sqrt(3.0) / 2.0;
        index.assign((2 * R + 1) * (2 * R + 1), -1);
        for (int a = -R; a <= R; a++)
            for (int b = -R; b <= R; b++) {
                if (std::abs(a + b) > R) continue;
                xy.push_back((float)((double)a + 0.5 * (double)b));
                xy.push_back((float)((double)b * s32));
                index[(a + R) * (2 * R + 1) + (b + R)] = n++;
            }
    }
    int at(int a, int b) const {
        if (a < -R || a > R || b < -R || b > R) return -1;
        return index[(a + R) * (2 * R + 1) + (b + R)];
    }
};

// Quantise one row; writes codes/scales and the dequantised row (float).
void pack_row(const float* w, int cols, const Codebook& cb, uint8_t* codes, uint16_t* scales, float* deq) {
    const double s32 = std::sqrt(3.0) / 2.0;
    const int R = cb.R;
    for (int blk = 0; blk < cols / 64; blk++) {
        const float* wb = w + (size_t)blk * 64;
        double A[32], B[32], M = 0.0;
        for (int p = 0; p < 32; p++) {
            double u = wb[2 * p], v = wb[2 * p + 1];
            double b = v / s32, a = u - 0.5 * b;
            A[p] = a; B[p] = b;
            double h = std::max(std::fabs(a), std::max(std::fabs(b), std::fabs(a + b)));
            M = std::max(M, h);
        }
        double s = M / (double)R;
        uint16_t s16 = float_to_half((float)s);
        if ((double)half_to_float(s16) < s && s16 < 0x7BFFu) s16++;   // round up
        scales[blk] = s16;
        const double sd = (double)half_to_float(s16);
        for (int p = 0; p < 32; p++) {
            int best = -1;
            if (sd > 0.0) {
                double a = A[p] / sd, b = B[p] / sd;
                double fa = std::floor(a), fb = std::floor(b), bd = 0.0;
                for (int c = 0; c < 4; c++) {
                    int ca = (int)fa + (c & 1), cb2 = (int)fb + (c >> 1);
                    int id = cb.at(ca, cb2);
                    if (id < 0) continue;
                    double dx = (a - ca) + 0.5 * (b - cb2), dy = s32 * (b - cb2);
                    double d = dx * dx + dy * dy;
                    if (best < 0 || d < bd) { best = id; bd = d; }
                }
                if (best < 0) {   // numerically on the hexagon rim: scan the book
                    double bdd = 0.0;
                    for (int i = 0; i < cb.n; i++) {
                        double dx = a + 0.5 * b - cb.xy[2 * i], dy = s32 * b - cb.xy[2 * i + 1];
                        double d = dx * dx + dy * dy;
                        if (best < 0 || d < bdd) { best = i; bdd = d; }
                    }
                }
            } else {
                best = cb.at(0, 0);
            }
            codes[blk * 32 + p] = (uint8_t)best;
            const float sf = half_to_float(s16);
            deq[blk * 64 + 2 * p] = cb.xy[2 * best] * sf;
            deq[blk * 64 + 2 * p + 1] = cb.xy[2 * best + 1] * sf;
        }
    }
}

void orthonormalize(std::vector<double>& M, int64_t n, int k, std::vector<double>* Rout) {
    // columns of M (n x k, row-major) by modified Gram-Schmidt, sequential sums
    if (Rout) Rout->assign((size_t)k * k, 0.0);
    for (int j = 0; j < k; j++) {
        for (int i = 0; i < j; i++) {
            double d = 0.0;
            for (int64_t r = 0; r < n; r++) d += M[r * k + i] * M[r * k + j];
            for (int64_t r = 0; r < n; r++) M[r * k + j] -= d * M[r * k + i];
            if (Rout) (*Rout)[i * k + j] = d;
        }
        double nrm = 0.0;
        for (int64_t r = 0; r < n; r++) nrm += M[r * k + j] * M[r * k + j];
        nrm = std::sqrt(nrm);
        if (Rout) (*Rout)[j * k + j] = nrm;
        double inv = nrm > 0.0 ? 1.0 / nrm : 0.0;
        for (int64_t r = 0; r < n; r++) M[r * k + j] *= inv;
    }
}

}  // namespace

extern "C" {

int gsdp_codebook(int radius, float* xy, int8_t* r01) {
    Codebook cb(radius);
    int n = 0;
    for (int a = -radius; a <= radius; a++)
        for (int b = -radius; b <= radius; b++) {
            if (std::abs(a + b) > radius) continue;
            if (xy) { xy[2 * n] = cb.xy[2 * n]; xy[2 * n + 1] = cb.xy[2 * n + 1]; }
            if (r01) { r01[2 * n] = (int8_t)a; r01[2 * n + 1] = (int8_t)b; }
            n++;
        }
    return n;
}

// n bf16-representable float32 values ~N(0, sigma) for (seed, stream).
void gsdp_synth_bf16(uint64_t seed, uint64_t stream, int64_t offset, int64_t n, float sigma, float* out) {
    const uint64_t key = stream_key(seed, stream);
    const float c = sigma / 65536.0f;
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = round_bf16((float)ih12(key, offset + i) * c);
}

// Same distribution rounded to fp16 bits (the embedding table).
void gsdp_synth_f16(uint64_t seed, uint64_t stream, int64_t offset, int64_t n, float sigma, uint16_t* out) {
    const uint64_t key = stream_key(seed, stream);
    const float c = sigma / 65536.0f;
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = float_to_half((float)ih12(key, offset + i) * c);
}

// Encode W [rows, cols] (row-major float32).  kink arrays need capacity
// rows * kinks_per_row.  Returns the number of kinks, or a negative error:
//   -1 unsupported radius, -2 cols not a positive multiple of 64,
//   -3 k_dim outside 0..16, -4 cols > 65536 (kink columns are u16).
int64_t gsdp_pack(const float* W, int rows, int cols, int radius, int k_dim, int kinks_per_row,
                  int lr_iters, uint8_t* codes, uint16_t* scales, uint32_t* row_ptr,
                  uint16_t* kink_cols, float* kink_deltas, uint16_t* U, float* S, uint16_t* Vt) {
    if (radius < 1 || radius > 8) return -1;
    if (cols <= 0 || cols % 64) return -2;
    if (k_dim < 0 || k_dim > 16) return -3;
    if (cols > 65536) return -4;
    const Codebook cb(radius);
    const bool need_res = k_dim > 0;
    std::vector<float> E(need_res ? (size_t)rows * cols : 0);
    std::vector<int> nk_row(rows, 0);
    const int kpr = std::max(0, std::min(kinks_per_row, cols));

    #pragma omp parallel
    {
        std::vector<float> deq(cols);
        std::vector<int> order(cols);
        #pragma omp for schedule(static)
        for (int r = 0; r < rows; r++) {
            const float* w = W + (size_t)r * cols;
            pack_row(w, cols, cb, codes + (size_t)r * cols / 2, scales + (size_t)r * cols / 64, deq.data());
            int nk = 0;
            if (kpr > 0) {
                for (int c = 0; c < cols; c++) order[c] = c;
                auto key = [&](int c) { return std::fabs(w[c] - deq[c]); };
                std::partial_sort(order.begin(), order.begin() + kpr, order.end(),
                                  [&](int x, int y) { float kx = key(x), ky = key(y); return kx > ky || (kx == ky && x < y); });
                std::sort(order.begin(), order.begin() + kpr);
                for (int i = 0; i < kpr; i++) {
                    int c = order[i];
                    float d = w[c] - deq[c];
                    if (d == 0.0f) continue;
                    kink_cols[(size_t)r * kpr + nk] = (uint16_t)c;
                    kink_deltas[(size_t)r * kpr + nk] = d;
                    deq[c] += d;
                    nk++;
                }
            }
            nk_row[r] = nk;
            if (need_res)
                for (int c = 0; c < cols; c++) E[(size_t)r * cols + c] = w[c] - deq[c];
        }
    }
    // compact the kink lists into CSR order
    int64_t total = 0;
    row_ptr[0] = 0;
    for (int r = 0; r < rows; r++) {
        if (kpr > 0 && total != (int64_t)r * kpr) {
            std::memmove(kink_cols + total, kink_cols + (size_t)r * kpr, nk_row[r] * sizeof(uint16_t));
            std::memmove(kink_deltas + total, kink_deltas + (size_t)r * kpr, nk_row[r] * sizeof(float));
        }
        total += nk_row[r];
        row_ptr[r + 1] = (uint32_t)total;
    }
    if (!need_res) return total;

    // rank-k factorisation of E by subspace iteration
    const int k = k_dim;
    std::vector<double> Q((size_t)cols * k), Y((size_t)rows * k);
    const uint64_t key = stream_key(0x5EEDull, (uint64_t)rows * 131071ull + (uint64_t)cols);
    for (int64_t i = 0; i < (int64_t)cols * k; i++)
        Q[i] = (double)(splitmix64(key + (uint64_t)i) >> 11) * (1.0 / 9007199254740992.0) - 0.5;
    orthonormalize(Q, cols, k, nullptr);
    auto mulEQ = [&]() {
        #pragma omp parallel for schedule(static)
        for (int r = 0; r < rows; r++) {
            double acc[16] = {0};
            const float* e = E.data() + (size_t)r * cols;
            for (int c = 0; c < cols; c++)
                for (int j = 0; j < k; j++) acc[j] += (double)e[c] * Q[(size_t)c * k + j];
            for (int j = 0; j < k; j++) Y[(size_t)r * k + j] = acc[j];
        }
    };
    for (int it = 0; it < lr_iters; it++) {
        mulEQ();
        orthonormalize(Y, rows, k, nullptr);
        std::fill(Q.begin(), Q.end(), 0.0);
        // Q = E^T Y; each column sums over rows in order (deterministic)
        #pragma omp parallel for schedule(static)
        for (int cb0 = 0; cb0 < cols; cb0 += 64) {
            const int ce = std::min(cols, cb0 + 64);
            for (int r = 0; r < rows; r++) {
                const float* e = E.data() + (size_t)r * cols;
                for (int c = cb0; c < ce; c++)
                    for (int j = 0; j < k; j++) Q[(size_t)c * k + j] += (double)e[c] * Y[(size_t)r * k + j];
            }
        }
        orthonormalize(Q, cols, k, nullptr);
    }
    mulEQ();
    std::vector<double> Rm;
    orthonormalize(Y, rows, k, &Rm);   // Y = Uq * Rm
    for (int j = 0; j < k; j++) {
        // row j of Rm * Q^T
        double nrm = 0.0;
        std::vector<double> v(cols);
        for (int c = 0; c < cols; c++) {
            double d = 0.0;
            for (int i = 0; i < k; i++) d += Rm[j * k + i] * Q[(size_t)c * k + i];
            v[c] = d;
            nrm += d * d;
        }
        nrm = std::sqrt(nrm);
        S[j] = (float)nrm;
        const double inv = nrm > 0.0 ? 1.0 / nrm : 0.0;
        for (int c = 0; c < cols; c++) Vt[(size_t)j * cols + c] = float_to_half((float)(v[c] * inv));
    }
    for (int r = 0; r < rows; r++)
        for (int j = 0; j < k; j++) U[(size_t)r * k + j] = float_to_half((float)Y[(size_t)r * k + j]);
    return total;
}

}  // extern "C"
