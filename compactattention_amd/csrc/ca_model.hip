// Fused element-wise kernels of the Llama integration (rotary embedding, RMSNorm, SwiGLU
// product).  They have no counterpart in the reference's _C_compactattn; they replace chains
// of PyTorch element-wise kernels (casts, rotate_half's negate + concatenate, multiplies,
// adds) around the compactattn layers with one pass each.  bf16 in and out, fp32 math.
//
// Numerics:
//  - rotary: out = bf16(q * cos + rotate_half(q) * sin), every product and the sum rounded
//    to fp32 separately (-ffp-contract=off) -- the same operations, in the same order, as
//    apply_rotary_pos_emb in fp32 (modeling_llama_common.py), so the result is bit-identical;
//  - RMSNorm: y = bf16(w * bf16(x * (1 / sqrt(mean(x^2) + eps)))), the transformers formula;
//    the mean's summation order is this kernel's own.  The residual form first adds the
//    residual in bf16 (x + r rounded once, as the decoder's residual + h) and normalises
//    that sum, returning both;
//  - SwiGLU: out = bf16(bf16(silu(g)) * u), silu in fp32.

#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {
namespace {

typedef uint16_t u16x8_t __attribute__((ext_vector_type(8)));

// One thread per 8 elements of a head row: lanes 0-7 hold d = 0..63 (their rotate partner
// d + 64 is read alongside), lanes 8-15 hold d = 64..127.  blockIdx.x is the token row
// (b * L + t), so a workgroup covers 16 heads of one token and the thread's head and chunk
// come from its index without divisions.
struct RopeParams {
    const uint16_t* x;
    int64_t xsb, xst, xsh;
    uint16_t* y;
    int64_t ysb, yst, ysh;
    const float* cos;  // [L, 128] rows for the L positions, row stride 128
    const float* sin;
    int B, L, H;
};

__global__ __launch_bounds__(256) void rope_kernel(RopeParams p) {
    const int bt = blockIdx.x;
    const int idx = blockIdx.y * 256 + threadIdx.x;
    const int h = idx >> 4;
    if (h >= p.H) return;
    const int c = idx & 15;  // 8-element chunk of the 128-wide row
    const int b = bt / p.L;
    const int t = bt - b * p.L;
    const uint16_t* xr = p.x + b * p.xsb + (int64_t)t * p.xst + (int64_t)h * p.xsh;
    uint16_t* yr = p.y + b * p.ysb + (int64_t)t * p.yst + (int64_t)h * p.ysh;
    const int d0 = 8 * c;
    const int dp = d0 < 64 ? d0 + 64 : d0 - 64;  // rotate_half partner
    const u16x8_t xv = *reinterpret_cast<const u16x8_t*>(xr + d0);
    const u16x8_t pv = *reinterpret_cast<const u16x8_t*>(xr + dp);
    const float4* cr = reinterpret_cast<const float4*>(p.cos + (int64_t)t * 128 + d0);
    const float4* sr = reinterpret_cast<const float4*>(p.sin + (int64_t)t * 128 + d0);
    const float4 c0 = cr[0], c1 = cr[1], s0 = sr[0], s1 = sr[1];
    const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    u16x8_t out;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float xi = bf16_to_f32(xv[i]);
        const float pi = bf16_to_f32(pv[i]);
        const float rot = d0 < 64 ? -pi : pi;
        const float a = xi * cv[i];
        const float bb = rot * sv[i];
        out[i] = f32_to_bf16(a + bb);
    }
    *reinterpret_cast<u16x8_t*>(yr + d0) = out;
}

// One workgroup of 256 threads per row; each thread sums the squares of its elements, the
// wave sums by xor shuffles and the four wave sums are added in a fixed order (the result
// is deterministic).  n must be a multiple of 8 (checked on the host).  With a residual the
// row is first s = bf16(x + r), written to s_out (the residual stream of the decoder layer),
// and the norm is taken of s; a thread re-reads only the elements it wrote itself, so s_out
// may alias x or r.  Up to kRmsKeep chunks per thread stay in registers between the passes.
struct RmsParams {
    const uint16_t* x;
    int64_t x_stride;
    const uint16_t* r;  // nullable
    int64_t r_stride;
    uint16_t* s;  // written when r is given
    int64_t s_stride;
    const uint16_t* w;
    uint16_t* y;
    int64_t y_stride;
    int n;
    float eps;
};

constexpr int kRmsKeep = 4;  // chunks per thread held in registers: rows up to 8192 elements

__global__ __launch_bounds__(256) void rmsnorm_kernel(RmsParams p) {
    __shared__ float part[4];
    const int64_t row = blockIdx.x;
    const uint16_t* xr = p.x + row * p.x_stride;
    uint16_t* yr = p.y + row * p.y_stride;
    const bool add = p.r != nullptr;
    const uint16_t* src = add ? p.s + row * p.s_stride : xr;
    // pass 1 over the thread's chunk i = 8 (t + 256 k): the (summed) row value, its square
    auto load = [&](int i, float& ss) {
        u16x8_t v = *reinterpret_cast<const u16x8_t*>(xr + i);
        if (add) {
            const u16x8_t rv = *reinterpret_cast<const u16x8_t*>(p.r + row * p.r_stride + i);
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = f32_to_bf16(bf16_to_f32(v[j]) + bf16_to_f32(rv[j]));
            *reinterpret_cast<u16x8_t*>(p.s + row * p.s_stride + i) = v;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float f = bf16_to_f32(v[j]);
            ss = __builtin_fmaf(f, f, ss);
        }
        return v;
    };
    float ss = 0.0f;
    u16x8_t keep[kRmsKeep];
#pragma unroll
    for (int k = 0; k < kRmsKeep; ++k) {
        const int i = threadIdx.x * 8 + k * 2048;
        if (i < p.n) keep[k] = load(i, ss);
    }
    for (int i = threadIdx.x * 8 + kRmsKeep * 2048; i < p.n; i += 2048) load(i, ss);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = (part[0] + part[1]) + (part[2] + part[3]);
    const float rstd = 1.0f / __builtin_sqrtf(total / static_cast<float>(p.n) + p.eps);
    auto store = [&](int i, const u16x8_t& v) {
        const u16x8_t wv = *reinterpret_cast<const u16x8_t*>(p.w + i);
        u16x8_t o;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float yn = bf16_to_f32(f32_to_bf16(bf16_to_f32(v[j]) * rstd));
            o[j] = f32_to_bf16(bf16_to_f32(wv[j]) * yn);
        }
        *reinterpret_cast<u16x8_t*>(yr + i) = o;
    };
#pragma unroll
    for (int k = 0; k < kRmsKeep; ++k) {
        const int i = threadIdx.x * 8 + k * 2048;
        if (i < p.n) store(i, keep[k]);
    }
    for (int i = threadIdx.x * 8 + kRmsKeep * 2048; i < p.n; i += 2048)
        store(i, *reinterpret_cast<const u16x8_t*>(src + i));
}

struct SwigluParams {
    const uint16_t* g;
    const uint16_t* u;
    uint16_t* y;
    int64_t rows;
    int n;
    int64_t g_stride, u_stride, y_stride;
};

__global__ __launch_bounds__(256) void swiglu_kernel(SwigluParams p) {
    const int64_t per_row = p.n / 8;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= p.rows * per_row) return;
    const int64_t row = gid / per_row;
    const int i = static_cast<int>(gid - row * per_row) * 8;
    const u16x8_t gv = *reinterpret_cast<const u16x8_t*>(p.g + row * p.g_stride + i);
    const u16x8_t uv = *reinterpret_cast<const u16x8_t*>(p.u + row * p.u_stride + i);
    u16x8_t o;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float g = bf16_to_f32(gv[j]);
        // silu(g) = g / (1 + e^-g); e^-g through exp2
        const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
        const float s = bf16_to_f32(f32_to_bf16(g / (1.0f + e)));
        o[j] = f32_to_bf16(s * bf16_to_f32(uv[j]));
    }
    *reinterpret_cast<u16x8_t*>(p.y + row * p.y_stride + i) = o;
}

}  // namespace

hipError_t launch_rope(const SeqAddr& x, const SeqAddr& y, const float* cos, const float* sin, int B, int L, int H,
                       hipStream_t stream) {
    RopeParams p;
    p.x = x.data;
    p.xsb = x.sb;
    p.xst = x.st;
    p.xsh = x.sh;
    p.y = y.data;
    p.ysb = y.sb;
    p.yst = y.st;
    p.ysh = y.sh;
    p.cos = cos;
    p.sin = sin;
    p.B = B;
    p.L = L;
    p.H = H;
    hipLaunchKernelGGL(rope_kernel, dim3(static_cast<unsigned>((int64_t)B * L), static_cast<unsigned>((H * 16 + 255) / 256)),
                       dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const uint16_t* x, int64_t x_stride, const uint16_t* r, int64_t r_stride, uint16_t* s,
                          int64_t s_stride, const uint16_t* w, uint16_t* y, int64_t y_stride, int64_t rows, int n,
                          float eps, hipStream_t stream) {
    RmsParams p;
    p.x = x;
    p.x_stride = x_stride;
    p.r = r;
    p.r_stride = r_stride;
    p.s = s;
    p.s_stride = s_stride;
    p.w = w;
    p.y = y;
    p.y_stride = y_stride;
    p.n = n;
    p.eps = eps;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_swiglu(const uint16_t* g, int64_t g_stride, const uint16_t* u, int64_t u_stride, uint16_t* y,
                         int64_t y_stride, int64_t rows, int n, hipStream_t stream) {
    SwigluParams p;
    p.g = g;
    p.u = u;
    p.y = y;
    p.rows = rows;
    p.n = n;
    p.g_stride = g_stride;
    p.u_stride = u_stride;
    p.y_stride = y_stride;
    const int64_t total = rows * (n / 8);
    hipLaunchKernelGGL(swiglu_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace ca
