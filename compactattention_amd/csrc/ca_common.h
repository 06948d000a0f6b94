// Shared device helpers for the compactattn HIP kernels (gfx950).
//
// Floating-point contract: the library is compiled with -ffp-contract=off.  Every fused
// multiply-add in the bit-reproducible kernels (pooling, gate projection, block scores,
// selection) is an explicit __builtin_fmaf; every other operation rounds on its own, and
// reductions run in the documented order.  Together with the in-house exp below this makes
// the fp32 block scores -- and therefore the selection masks and block tables -- identical
// to a CPU evaluation in the same order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/compactattn.h"

namespace ca {

constexpr int kD = CA_HEAD_DIM;   // head dim
constexpr int kBlock = CA_BLOCK;  // tokens per block / page

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// exp(x): Cody-Waite reduction n = rint(x log2 e), r = x - n*ln2 (ln2 split into a
// high part with zero trailing bits and a low part), degree-7 Taylor polynomial of e^r on
// |r| <= ln2/2 in Horner form, times 2^n from the exponent bits.  Inputs below -80 give 0
// (no subnormal results), above 88 give +inf.
__device__ __forceinline__ float exp_fixed(float x) {
    if (x != x) return x;
    if (x < -80.0f) return 0.0f;
    if (x > 88.0f) return __builtin_inff();
    const float n = __builtin_rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(n, -0x1.62e400p-1f, x);
    r = __builtin_fmaf(n, -0x1.7f7d1cp-20f, r);
    float p = 1.98412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333333e-3f);
    p = __builtin_fmaf(p, r, 4.16666667e-2f);
    p = __builtin_fmaf(p, r, 1.66666667e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ni = static_cast<int>(n);
    return p * __uint_as_float(static_cast<uint32_t>(ni + 127) << 23);
}

// Sum of 256 per-thread partials in the canonical order part[t] += part[t + s] for
// s = 128, 64, ..., 1 (blockDim.x must be 256; scratch holds 256 floats).  The result is
// returned to every thread.
__device__ __forceinline__ float tree256_sum(float v, float* scratch) {
    const int t = threadIdx.x;
    scratch[t] = v;
    __syncthreads();
#pragma unroll
    for (int s = 128; s >= 1; s >>= 1) {
        if (t < s) scratch[t] = scratch[t] + scratch[t + s];
        __syncthreads();
    }
    const float r = scratch[0];
    __syncthreads();
    return r;
}

__device__ __forceinline__ float block_max256(float v, float* scratch) {
    const int t = threadIdx.x;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    if ((t & 63) == 0) scratch[t >> 6] = v;
    __syncthreads();
    const float r = fmaxf(fmaxf(scratch[0], scratch[1]), fmaxf(scratch[2], scratch[3]));
    __syncthreads();
    return r;
}

__device__ __forceinline__ int block_sum256_int(int v, int* scratch) {
    const int t = threadIdx.x;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((t & 63) == 0) scratch[t >> 6] = v;
    __syncthreads();
    const int r = scratch[0] + scratch[1] + scratch[2] + scratch[3];
    __syncthreads();
    return r;
}

// Exclusive prefix over a 256-thread block (ascending thread order) and the block total.
__device__ __forceinline__ int block_exclusive_scan256(int v, int* scratch, int* total) {
    const int t = threadIdx.x;
    const int lane = t & 63;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63) scratch[t >> 6] = incl;
    __syncthreads();
    int wave_off = 0;
    for (int w = 0; w < (t >> 6); ++w) wave_off += scratch[w];
    *total = scratch[0] + scratch[1] + scratch[2] + scratch[3];
    __syncthreads();
    return wave_off + incl - v;
}

}  // namespace ca
