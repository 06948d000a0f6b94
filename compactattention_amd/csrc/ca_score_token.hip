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
// One workgroup of 8 waves per (request x Q head, query block).  The block's BS x 128 query
// tile sits in LDS, read by every wave as the A operand of v_mfma_f32_32x32x16_bf16 (tokens
// as M); the waves take 32-key tiles in turn, key means as the B operand (keys as N), so each
// lane ends with the scores of one key over 16 token rows per 32-token tile, and the max and
// the exp2 sum over the block's tokens take one lane-half exchange.  m and p go through LDS to
// the normalisation over the row.  A wave loads its key tile with whole 512-byte rows per
// instruction and stages it as bf16 through 8 KB of its own LDS (loads in the MFMA operand
// layout touch 32 rows per instruction and ran 68 against 47 us at config 2), with the next
// tile's loads in flight while it computes.  Every workgroup streams its KV row's whole
// key-mean row, so the workgroups are placed on the 8 XCDs by KV row: each XCD's L2 then
// holds the rows of its own workgroups only (config 2: one 1 MB row per XCD instead of all
// eight).  Tiles whose keys every token of the block sees skip the causal test.

#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {
namespace {

typedef __bf16 tm_bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 tm_bf16x4_t __attribute__((ext_vector_type(4)));
typedef float tm_f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kTmWaves = 8;

struct TokenMassParams {
    Shape s;          // B, Lq, Hq, Hkv, G; cap = key blocks per row of khat and scores
    SeqAddr q;
    const float* khat;
    int64_t khat_stride;  // blocks per row of khat (row = b*Hkv + hk)
    float sm_scale;       // scale * log2(e)
    PastBlocks pb;        // past blocks (of block_size tokens)
    float* scores;        // [B, Hq, Qb, cap]
    int qb_count;         // ceil(Lq / bs)
    int total;            // work items: B * Hq * qb_count, in (KV row, head of the group, query block) order
    int per_xcd;          // ceil(total / 8): XCD x takes items [x * per_xcd, (x + 1) * per_xcd)
};

__device__ __forceinline__ float tm_xor32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float tm_xor32_add(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// MT = 32-token tiles per query block (2 for 64-token blocks, 4 for 128).  LDS: the block's
// query tile (MT * 32 rows of 256 B, 16-byte chunk c of row r at chunk c ^ (r & 15)), then
// m[cap], pmass[cap] (each padded to a multiple of 4 floats), 16 floats of reductions and
// 8 KB of key tile per wave.
template <int MT>
__global__ __launch_bounds__(kTmWaves * 64) __attribute__((amdgpu_waves_per_eu(2))) void token_mass_kernel(TokenMassParams p) {
    extern __shared__ __attribute__((aligned(16))) float tm_lds[];
    const Shape& s = p.s;
    // workgroup L runs on XCD L % 8 (round-robin dispatch); it takes that XCD's (L / 8)-th item
    const int item = (blockIdx.x & 7) * p.per_xcd + (blockIdx.x >> 3);
    if (item >= p.total) return;
    const int qb = item % p.qb_count;
    const int rg = item / p.qb_count;  // (b * Hkv + hk) * G + g
    const int kvrow = rg / s.G;
    const int b = kvrow / s.Hkv;
    const int hk = kvrow - b * s.Hkv;
    const int h = hk * s.G + (rg - kvrow * s.G);
    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int l = tid & 63;
    const int n = l & 31;
    const int half = l >> 5;
    constexpr int BS = 32 * MT;
    const int P = p.pb.p[b];
    const int cap = s.cap;
    const int nk = P + p.qb_count;                      // key blocks of the request
    const int64_t start = (int64_t)P * BS;              // absolute position of query token 0
    const int64_t qmax = start + (int64_t)qb * BS + BS - 1;
    const int hi = (int)min((int64_t)nk, (qmax + 1 + BS - 1) / BS);
    uint8_t* qs = reinterpret_cast<uint8_t*>(tm_lds);
    const int cap4 = (cap + 3) & ~3;  // keeps the arrays after m and p 16-byte aligned
    float* mrow = tm_lds + BS * 64;
    float* prow = mrow + cap4;
    float* red = prow + cap4;

    // ---- the query tile into LDS (tokens past q_len are zero slots) ----
    for (int f = tid; f < BS * 16; f += kTmWaves * 64) {
        const int row = f >> 4, c = f & 15;
        const int t = qb * BS + row;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (t < s.Lq)
            v = *reinterpret_cast<const uint4*>(p.q.data + b * p.q.sb + (int64_t)t * p.q.st + (int64_t)h * p.q.sh + 8 * c);
        *reinterpret_cast<uint4*>(qs + row * 256 + ((c ^ (row & 15)) << 4)) = v;
    }
    __syncthreads();

    const float* krow = p.khat + ((int64_t)b * s.Hkv + hk) * p.khat_stride * kD;
    const int ntiles = (hi + 31) / 32;
    // each wave stages its key tile through its own 8 KB of LDS as bf16 (32 keys x 256 B,
    // 16-byte chunk c of key r at chunk c ^ (r & 15)): global loads take whole rows, 1 KB per
    // instruction, and the MFMA operands come back with one ds_read_b128 each
    uint8_t* kt = reinterpret_cast<uint8_t*>(red + 2 * kTmWaves) + w * 8192;
    // tile j's key means: 16 float4 per lane, whole rows per instruction (lane l takes float4
    // l & 31 of keys (l >> 5) + 2 i), all 16 loads issued back to back through a buffer
    // resource whose range ends at key hi: keys past it read as zeros (their columns of the
    // scores are dropped by the kvalid test below), and four 4 KB steps of the vector offset
    // with the 0 / 1 / 2 / 3 KB instruction offsets address the 16 loads.
    float4 kv[16];
    const int kh = l >> 5, c4 = l & 31;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(krow), 0, hi * kD * 4, 0x00020000);
    const int lane_off = kh * (kD * 4) + c4 * 16;
    auto issue_tile = [&](int j) {
        if (j >= ntiles) return;
        const int tb = 32 * j * (kD * 4);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int vo = lane_off + tb + q * 4096;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                kv[4 * q + r] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(krs, vo + r * 1024, 0, 0));
        }
    };
    // LDS byte offsets of key kh + 2 i's float4 c4 (i < 8; key + 16 adds 4096 and keeps the swizzle)
    int soff[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int key = kh + 2 * i;
        soff[i] = key * 256 + (((c4 >> 1) ^ (key & 15)) << 4) + (c4 & 1) * 8;
    }
    // and of the MFMA operands: chunk 2 ks + half of row n (K) or row 32 mt + n (Q, + 8192 mt)
    int foff[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) foff[ks] = n * 256 + (((2 * ks + half) ^ (n & 15)) << 4);
    auto stage_tile = [&]() {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 v = kv[i];
            tm_bf16x4_t v4;  // bf16(meanK), round to nearest even
            v4[0] = static_cast<__bf16>(v.x);
            v4[1] = static_cast<__bf16>(v.y);
            v4[2] = static_cast<__bf16>(v.z);
            v4[3] = static_cast<__bf16>(v.w);
            *reinterpret_cast<tm_bf16x4_t*>(kt + soff[i & 7] + (i >> 3) * 4096) = v4;
        }
    };
    issue_tile(w);
    for (int j = w; j < ntiles; j += kTmWaves) {
        const int kb = 32 * j + n;
        const bool kvalid = kb < hi;
        stage_tile();
        issue_tile(j + kTmWaves);  // in flight while this tile computes
        tm_f32x16_t acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mt][i] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const tm_bf16x8_t kb8 = *reinterpret_cast<const tm_bf16x8_t*>(kt + foff[ks]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                // row 32 mt + n has the swizzle of row n (32 mt is a multiple of 16)
                const tm_bf16x8_t qa = *reinterpret_cast<const tm_bf16x8_t*>(qs + mt * 8192 + foff[ks]);
                acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa, kb8, acc[mt], 0, 0, 0);
            }
        }
        // lane (n, half) holds key kb over token rows 32 mt + 8 (r / 4) + 4 half + r % 4.
        // m = max_t s = max_t(acc) * sm_scale (sm_scale > 0), and exp2(s - m) is taken as
        // exp2(fma(acc, sm_scale, -m))
        const int64_t q0 = start + (int64_t)qb * BS;            // position of the block's first token
        const bool all_see = (int64_t)(32 * j + 31) * BS + BS - 1 <= q0;  // every token sees every key
        float m = -__builtin_inff();
        float sum = 0.0f;
        if (all_see) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) m = fmaxf(m, acc[mt][r]);
            m = tm_xor32_max(m) * p.sm_scale;
            const float mneg = -m;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) sum += __builtin_amdgcn_exp2f(__builtin_fmaf(acc[mt][r], p.sm_scale, mneg));
        } else {
            // token t sees the key block when q0 + t >= its last token kb * BS + BS - 1
            const int tmin = (int)max((int64_t)0, min((int64_t)BS, (int64_t)kb * BS + BS - 1 - q0));
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int t = 32 * mt + 8 * (r >> 2) + 4 * half + (r & 3);
                    if (t < tmin) acc[mt][r] = -__builtin_inff();
                    m = fmaxf(m, acc[mt][r]);
                }
            m = tm_xor32_max(m) * p.sm_scale;  // -inf: no token of the block sees the key
            const float mneg = -m;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float a = acc[mt][r];
                    sum += a == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(__builtin_fmaf(a, p.sm_scale, mneg));
                }
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
    float M = red[0];
#pragma unroll
    for (int i = 1; i < kTmWaves; ++i) M = fmaxf(M, red[i]);
    float part = 0.0f;
    for (int kb = tid; kb < nk; kb += kTmWaves * 64) {
        const float mk = mrow[kb];
        const float sc = mk != -__builtin_inff() ? prow[kb] * __builtin_amdgcn_exp2f(mk - M) : 0.0f;
        prow[kb] = sc;
        part += sc;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) part += __shfl_xor(part, o, 64);
    if (l == 0) red[kTmWaves + w] = part;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kTmWaves; ++i) tot += red[kTmWaves + i];
    const float denom = tot + 1e-9f;
    float* out = p.scores + (((int64_t)b * s.Hq + h) * p.qb_count + qb) * cap;
    for (int kb = tid; kb < cap; kb += kTmWaves * 64) out[kb] = kb < nk ? prow[kb] / denom : 0.0f;
}

}  // namespace

size_t token_mass_lds_bytes(const Shape& s, int bs) {
    const size_t cap4 = ((size_t)s.cap + 3) & ~(size_t)3;
    return (size_t)bs * 256 + sizeof(float) * (2 * cap4 + 2 * kTmWaves) + 8192 * kTmWaves;
}

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
    p.qb_count = (s.Lq + bs - 1) / bs;
    p.total = p.qb_count * s.B * s.Hq;
    p.per_xcd = (p.total + 7) / 8;
    dim3 grid(8 * p.per_xcd);
    const size_t lds = token_mass_lds_bytes(s, bs);
    if (bs == 64)
        hipLaunchKernelGGL(token_mass_kernel<2>, grid, dim3(kTmWaves * 64), lds, stream, p);
    else
        hipLaunchKernelGGL(token_mass_kernel<4>, grid, dim3(kTmWaves * 64), lds, stream, p);
    return hipGetLastError();
}

}  // namespace ca
