// FlashPrefill block scores in the reference's per-token form, for gfx950.
//
// Reference: compact_attn/flashprefill_vendor/flashprefill_native_forward.py:98-207
// (compute_block_score_chunked with K_STRIDE = BLOCK_SIZE, as flash_prefill_select_chunked and
// flash_prefill_score_chunked_from_mean_k call it, :466-489,562-582) and normalize_scores
// (:365-374).  For request b, Q head h, query block qb (block_size tokens starting at query
// token 0) and key block kb < hi = min(ceil((q_max + 1) / BS), nk):
//   s[t, kb] = dot(q_t, bf16(meanK_kb)) * scale * log2(e)   when q_abs(t) >= kb*BS + BS - 1,
//              -inf otherwise,
//   m[kb]    = max_t s[t, kb],   p[kb] = sum_t exp2(s[t, kb] - m[kb])  (causal t only),
// over the block's BS token slots; slots past q_len hold q = 0 (the reference loads them as 0
// and keeps them, at absolute positions past the key range).  q_abs(t) = P*BS + qb*BS + t,
// q_max = P*BS + qb*BS + BS - 1, nk = P + ceil(q_len / BS).  Then, over kb of the row:
//   M = max_kb m,  score = p * exp2(m - M) where m > -inf (0 elsewhere),
//   score /= sum_kb score + 1e-9.
// The key means are rounded to bf16 as the reference stores them (mean_k has K's dtype) and
// the dot products run on bf16 MFMAs with fp32 accumulation, as tl.dot does; the row's sums
// use a fixed order of this kernel's own (the values agree with an fp64 evaluation to a few
// ulps, not bit for bit).
//
// One workgroup of 4 waves per (query block, request x Q head).  The block's BS x 128 query
// tile sits in every wave's registers as the A operand of v_mfma_f32_32x32x16_bf16 (tokens as
// M); the waves take 32-key tiles in turn, key means as the B operand (keys as N), so each
// lane ends with the scores of one key over 16 token rows per 32-token tile, and the max and
// the exp2 sum over the block's tokens take one lane-half exchange.  m and p go through LDS to
// the normalisation over the row.

#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {
namespace {

typedef __bf16 tm_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float tm_f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kTmWaves = 4;

struct TokenMassParams {
    Shape s;          // B, Lq, Hq, Hkv, G; cap = key blocks per row of khat and scores
    SeqAddr q;
    const float* khat;
    int64_t khat_stride;  // blocks per row of khat (row = b*Hkv + hk)
    float sm_scale;       // scale * log2(e)
    PastBlocks pb;        // past blocks (of block_size tokens)
    float* scores;        // [B, Hq, Qb, cap]
    int bs;               // block size: 64 or 128
    int qb_count;         // ceil(Lq / bs)
};

__device__ __forceinline__ float tm_xor32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float tm_xor32_add(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// MT = 32-token tiles per query block (2 for 64-token blocks, 4 for 128)
template <int MT>
__global__ __launch_bounds__(kTmWaves * 64) void token_mass_kernel(TokenMassParams p) {
    extern __shared__ float tm_lds[];  // m[cap], then pmass[cap], then 8 floats of reductions
    const Shape& s = p.s;
    const int qb = blockIdx.x;
    const int bh = blockIdx.y;
    const int b = bh / s.Hq;
    const int h = bh - b * s.Hq;
    const int hk = h / s.G;
    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int l = tid & 63;
    const int n = l & 31;
    const int half = l >> 5;
    const int BS = p.bs;
    const int P = p.pb.p[b];
    const int cap = s.cap;
    const int nk = P + p.qb_count;                      // key blocks of the request
    const int64_t start = (int64_t)P * BS;              // absolute position of query token 0
    const int64_t qmax = start + (int64_t)qb * BS + BS - 1;
    const int hi = (int)min((int64_t)nk, (qmax + 1 + BS - 1) / BS);
    float* mrow = tm_lds;
    float* prow = tm_lds + cap;
    float* red = tm_lds + 2 * cap;

    // ---- the query tile: A[m = token][k = d] ----
    tm_bf16x8_t qa[MT][8];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int t = qb * BS + 32 * mt + n;  // token of the chunk
        const bool valid = t < s.Lq;
        const uint16_t* qp = p.q.data + b * p.q.sb + (int64_t)(valid ? t : 0) * p.q.st + (int64_t)h * p.q.sh + 8 * half;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            if (valid) {
                qa[mt][ks] = *reinterpret_cast<const tm_bf16x8_t*>(qp + 16 * ks);
            } else {
                for (int i = 0; i < 8; ++i) qa[mt][ks][i] = static_cast<__bf16>(0.0f);
            }
        }
    }

    const float* krow = p.khat + ((int64_t)b * s.Hkv + hk) * p.khat_stride * kD;
    const int ntiles = (hi + 31) / 32;
    for (int j = w; j < ntiles; j += kTmWaves) {
        const int kb = 32 * j + n;
        const bool kvalid = kb < hi;
        tm_f32x16_t acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mt][i] = 0.0f;
        const float* kp = krow + (int64_t)(kvalid ? kb : 0) * kD + 8 * half;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            float4 lo = make_float4(0.f, 0.f, 0.f, 0.f), hi4 = lo;
            if (kvalid) {
                lo = *reinterpret_cast<const float4*>(kp + 16 * ks);
                hi4 = *reinterpret_cast<const float4*>(kp + 16 * ks + 4);
            }
            tm_bf16x8_t kb8;  // bf16(meanK), round to nearest even
            kb8[0] = static_cast<__bf16>(lo.x);
            kb8[1] = static_cast<__bf16>(lo.y);
            kb8[2] = static_cast<__bf16>(lo.z);
            kb8[3] = static_cast<__bf16>(lo.w);
            kb8[4] = static_cast<__bf16>(hi4.x);
            kb8[5] = static_cast<__bf16>(hi4.y);
            kb8[6] = static_cast<__bf16>(hi4.z);
            kb8[7] = static_cast<__bf16>(hi4.w);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[mt][ks], kb8, acc[mt], 0, 0, 0);
        }
        // lane (n, half) holds key kb over token rows 32 mt + 8 (r / 4) + 4 half + r % 4
        const int64_t kend = (int64_t)kb * BS + BS - 1;  // last token of the key block
        float m = -__builtin_inff();
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = 32 * mt + 8 * (r >> 2) + 4 * half + (r & 3);
                const bool causal = start + (int64_t)qb * BS + t >= kend;
                const float v = causal ? acc[mt][r] * p.sm_scale : -__builtin_inff();
                acc[mt][r] = v;
                m = fmaxf(m, v);
            }
        m = tm_xor32_max(m);
        float sum = 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float v = acc[mt][r];
                sum += v == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(v - m);
            }
        sum = tm_xor32_add(sum);
        if (half == 0 && kb < cap) {
            mrow[kb] = kvalid ? m : -__builtin_inff();
            prow[kb] = kvalid ? sum : 0.0f;
        }
    }
    // key blocks the reference never scores (hi .. cap) read as unscored
    for (int kb = 32 * ntiles + tid; kb < cap; kb += kTmWaves * 64) {
        mrow[kb] = -__builtin_inff();
        prow[kb] = 0.0f;
    }
    __syncthreads();

    // ---- normalize_scores over the row's key blocks ----
    float mx = -__builtin_inff();
    for (int kb = tid; kb < nk; kb += kTmWaves * 64) mx = fmaxf(mx, mrow[kb]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (l == 0) red[w] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float part = 0.0f;
    for (int kb = tid; kb < nk; kb += kTmWaves * 64) {
        const float mk = mrow[kb];
        const float sc = mk != -__builtin_inff() ? prow[kb] * __builtin_amdgcn_exp2f(mk - M) : 0.0f;
        prow[kb] = sc;
        part += sc;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) part += __shfl_xor(part, o, 64);
    __syncthreads();  // red[] reused
    if (l == 0) red[4 + w] = part;
    __syncthreads();
    const float denom = ((red[4] + red[5]) + (red[6] + red[7])) + 1e-9f;
    float* out = p.scores + (((int64_t)b * s.Hq + h) * p.qb_count + qb) * cap;
    for (int kb = tid; kb < cap; kb += kTmWaves * 64) out[kb] = kb < nk ? prow[kb] / denom : 0.0f;
}

}  // namespace

size_t token_mass_lds_bytes(const Shape& s) { return sizeof(float) * (2 * (size_t)s.cap + 8); }

hipError_t launch_token_mass(const Shape& s, const SeqAddr& q, const float* khat, int64_t khat_stride, int bs,
                             float scale, const PastBlocks& pb, float* scores, hipStream_t stream) {
    TokenMassParams p;
    p.s = s;
    p.q = q;
    p.khat = khat;
    p.khat_stride = khat_stride;
    p.sm_scale = scale * 1.4426950408889634f;
    p.pb = pb;
    p.scores = scores;
    p.bs = bs;
    p.qb_count = (s.Lq + bs - 1) / bs;
    dim3 grid(p.qb_count, s.B * s.Hq);
    const size_t lds = token_mass_lds_bytes(s);
    if (bs == 64)
        hipLaunchKernelGGL(token_mass_kernel<2>, grid, dim3(kTmWaves * 64), lds, stream, p);
    else
        hipLaunchKernelGGL(token_mass_kernel<4>, grid, dim3(kTmWaves * 64), lds, stream, p);
    return hipGetLastError();
}

}  // namespace ca
