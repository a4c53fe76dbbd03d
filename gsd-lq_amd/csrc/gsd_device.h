// gsd_device.h -- device helpers shared by the kernels of libgsdhip.so:
// fp16 conversions, wave / row reductions in VALU (DPP, permlane swaps),
// the greedy top-2 merge and the LDS-only workgroup barrier.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gsd {
namespace {

// Float max for values that are never NaN (scores, -inf masks, partial
// maxima): the IEEE maximum, one v_maximum3_f32 with no canonicalising moves
// in front of values that come from DPP, permlane swaps or memory, which
// fmaxf (NaN-ignoring) needs for each such operand.
__device__ __forceinline__ float fmax_nc(float a, float b) { return __builtin_elementwise_maximum(a, b); }
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

__device__ __forceinline__ float swap_add32(float a, float b, bool upper) {
    // lanes 0-31 get a(lo)+a(hi), lanes 32-63 get b(lo)+b(hi)
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    (void)upper;
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap_add16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float row16_sum(float v) {
    v += __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0xB1, 0xF, 0xF, true));   // quad_perm 1,0,3,2
    v += __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0x4E, 0xF, 0xF, true));   // quad_perm 2,3,0,1
    v += __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0x141, 0xF, 0xF, true));  // row_half_mirror
    v += __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0x140, 0xF, 0xF, true));  // row_mirror
    return v;
}

__device__ __forceinline__ float row16_max(float v) {
    v = fmax_nc(v, __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0xB1, 0xF, 0xF, true)));
    v = fmax_nc(v, __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0x4E, 0xF, 0xF, true)));
    v = fmax_nc(v, __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0x141, 0xF, 0xF, true)));
    v = fmax_nc(v, __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0x140, 0xF, 0xF, true)));
    return v;
}
// Whole-wave sum / max in every lane, in VALU only (row DPP, then the
// 16- and 32-lane swaps); all 64 lanes must be active.
__device__ __forceinline__ float wave_sum_valu(float v) {
    v = row16_sum(v);
    v = swap_add16(v, v);
    return swap_add32(v, v, false);
}
// Whole-wave max of values >= 0 (no NaN) in every lane: unsigned compares of
// the bit patterns order such floats, and need none of the canonicalising
// moves that float max inserts after each DPP or swap.
__device__ __forceinline__ float wave_max_nonneg(float v) {
    unsigned u = __float_as_uint(v);
    u = max(u, (unsigned)__builtin_amdgcn_mov_dpp((int)u, 0xB1, 0xF, 0xF, true));
    u = max(u, (unsigned)__builtin_amdgcn_mov_dpp((int)u, 0x4E, 0xF, 0xF, true));
    u = max(u, (unsigned)__builtin_amdgcn_mov_dpp((int)u, 0x141, 0xF, 0xF, true));
    u = max(u, (unsigned)__builtin_amdgcn_mov_dpp((int)u, 0x140, 0xF, 0xF, true));
    auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    u = max(r[0], r[1]);
    r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(max(r[0], r[1]));
}
__device__ __forceinline__ float wave_max_valu(float v) {
    v = row16_max(v);
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmax_nc(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmax_nc(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Code tiles of the matrix-core matvec: a 16-row x 128-column tile of codes,
// one 16-code word per lane (lane l: row l & 15).  Codebooks of more than 128
// points (radius 7-8) use one byte per code: 1024 bytes, lane l at byte 16 l.
// Codebooks of at most 128 points (radius <= 6) use 7 bits per code: 896
// bytes, lane pair i owning bytes 28 i .. 28 i + 27, the 16 codes of lane 2 i
// as a 112-bit little-endian field (code j = bits 7 j .. 7 j + 6) at byte
// 28 i and those of lane 2 i + 1 at byte 28 i + 14.  Lane 2 i loads 16 bytes
// at 28 i and lane 2 i + 1 at 28 i + 12 (4-byte aligned), so an odd lane's
// field starts at bit 16 of its word until align7 shifts it down.
constexpr int kTileU8 = 1024, kTile7 = 896;
__device__ __forceinline__ int tile_bytes(bool b7) { return b7 ? kTile7 : kTileU8; }
__device__ __forceinline__ uint32_t tile_lane_off(bool b7, int lane) {
    return b7 ? 28u * (uint32_t)(lane >> 1) + 12u * (uint32_t)(lane & 1) : 16u * (uint32_t)lane;
}
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ uint4 tile_load(const unsigned char* p) {   // p = tile + tile_lane_off
    const u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
// 7-bit word with the lane's field moved to bit 0 (sh = 16 on odd lanes, 0 on even)
__device__ __forceinline__ void align7(uint32_t (&w)[4], uint32_t sh) {
    w[0] = __builtin_amdgcn_alignbit(w[1], w[0], sh);
    w[1] = __builtin_amdgcn_alignbit(w[2], w[1], sh);
    w[2] = __builtin_amdgcn_alignbit(w[3], w[2], sh);
    w[3] = w[3] >> sh;
}
// code j (a constant after unrolling) of an aligned 7-bit word at bits 8 .. 14
__device__ __forceinline__ uint32_t win7(const uint32_t (&w)[4], int j) {
    if (j == 0) return w[0] << 8;
    if (j == 1) return w[0] << 1;
    const int s = 7 * j - 8, d = s >> 5, sh = s & 31;
    return d == 3 ? w[3] >> sh : __builtin_amdgcn_alignbit(w[d + 1], w[d], sh);
}
// code j of a lane's word (u8 word, or 7-bit word after align7)
__device__ __forceinline__ uint32_t code_of(const uint32_t (&w)[4], int j, bool b7) {
    return b7 ? (win7(w, j) >> 8) & 0x7Fu : (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
}
// LDS address code * 256 + lane * 4 of code j (lane_off = lane * 4): the
// entry of the lane's own copy of the codebook
__device__ __forceinline__ uint32_t code_addr(const uint32_t (&w)[4], int j, uint32_t lane_off, bool b7) {
    return b7 ? ((win7(w, j) & 0x7F00u) | lane_off)
              : __builtin_amdgcn_perm(w[j >> 2], lane_off, 0x0C0C0400u + ((uint32_t)(j & 3) << 8));
}

__device__ __forceinline__ float dpp_sum8(float v) {    // sum within 8-lane half-rows
    v += __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0xB1, 0xF, 0xF, true));
    v += __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0x4E, 0xF, 0xF, true));
    v += __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0x141, 0xF, 0xF, true));
    return v;
}
template <int LPP>
__device__ __forceinline__ float lane_group_sum(float v) {   // sum over LPP consecutive lanes
    if (LPP == 8) return dpp_sum8(v);
    v = row16_sum(v);
    if (LPP == 32) v = swap_add16(v, v);
    return v;
}
__device__ __forceinline__ float wave_allsum(float v) {
    v = row16_sum(v);
    v = swap_add16(v, v);
    return swap_add32(v, v, false);
}
__device__ __forceinline__ float wave_allmax(float v) {
    v = fmax_nc(v, __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0xB1, 0xF, 0xF, true)));
    v = fmax_nc(v, __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0x4E, 0xF, 0xF, true)));
    v = fmax_nc(v, __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0x141, 0xF, 0xF, true)));
    v = fmax_nc(v, __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0x140, 0xF, 0xF, true)));
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmax_nc(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmax_nc(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// sum over the position slots of a wave (lanes with equal lane % LPP)
template <int LPP>
__device__ __forceinline__ float slot_sum(float v) {
    if (LPP == 8) v += __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), 0x128, 0xF, 0xF, true));  // row_ror:8
    if (LPP <= 16) v = swap_add16(v, v);
    return swap_add32(v, v, false);
}
__device__ __forceinline__ void unpack8(const uint4 w, float (&f)[8]) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 8; e++) f[e] = h2f((uint16_t)(u[e >> 1] >> (16 * (e & 1))));
}

// greedy argmax: nan -> -1e4, +inf -> 100, -inf -> -1e4, first index wins
__device__ __forceinline__ float clean(float v) {
    if (v != v) return -1e4f;
    if (v == INFINITY) return 100.f;
    if (v == -INFINITY) return -1e4f;
    return v;
}

// (value, index, runner-up) merge: higher value wins, lower index on ties
struct Top2 {
    float v1, v2;
    int i1;
};
__device__ __forceinline__ Top2 merge(Top2 a, Top2 b) {
    Top2 r;
    if (b.v1 > a.v1 || (b.v1 == a.v1 && b.i1 < a.i1)) {
        r.v1 = b.v1; r.i1 = b.i1; r.v2 = fmaxf(a.v1, b.v2);
    } else {
        r.v1 = a.v1; r.i1 = a.i1; r.v2 = fmaxf(a.v2, b.v1);
    }
    return r;
}

typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// Workgroup barrier for LDS traffic only.  __syncthreads() is a workgroup
// fence plus s_barrier, and on this target the fence waits for every
// outstanding vector memory operation of the wave (vmcnt(0)), which would
// drain the prefetched code loads at each barrier.  Here each wave waits for
// its own LDS operations (lgkmcnt(0); vmcnt and expcnt left at their maxima:
// 0xC07F) and then meets the others; the empty asm statements keep the
// compiler from moving memory accesses across.
__device__ __forceinline__ void lds_barrier() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

}  // namespace
}  // namespace gsd
