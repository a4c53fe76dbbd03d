// gsd_device.h -- device helpers shared by the kernels of libgsdhip.so:
// fp16 conversions, wave / row reductions in VALU (DPP, permlane swaps),
// the greedy top-2 merge and the LDS-only workgroup barrier.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

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
    v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
    v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
    v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
    v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x140, 0xF, 0xF, false));  // row_mirror
    return v;
}

__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x140, 0xF, 0xF, false)));
    return v;
}
// Whole-wave sum / max in every lane, in VALU only (row DPP, then the
// 16- and 32-lane swaps); all 64 lanes must be active.
__device__ __forceinline__ float wave_sum_valu(float v) {
    v = row16_sum(v);
    v = swap_add16(v, v);
    return swap_add32(v, v, false);
}
__device__ __forceinline__ float wave_max_valu(float v) {
    v = row16_max(v);
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float dpp_sum8(float v) {    // sum within 8-lane half-rows
    v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0xB1, 0xF, 0xF, false));
    v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x4E, 0xF, 0xF, false));
    v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x141, 0xF, 0xF, false));
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
    v = fmaxf(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x140, 0xF, 0xF, false)));
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// sum over the position slots of a wave (lanes with equal lane % LPP)
template <int LPP>
__device__ __forceinline__ float slot_sum(float v) {
    if (LPP == 8) v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x128, 0xF, 0xF, false));  // row_ror:8
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
