// Cache fill, pooled summaries, block scoring + selection and Block-Union compaction
// kernels for gfx950.
//
// Reference behaviour (paths relative to the reference repository):
//  - cache fill / mean-K: compact_attn/flashprefill_vendor/flashprefill_native_forward.py:44-95,
//    transformers DynamicCache.update as used at compact_attn/prefill_sparse/llama/
//    modeling_llama_seerattn_chunked_dense.py:518-536.
//  - gate projection + block RoPE: compact_attn/prefill_sparse/attn_gate.py:20-34,113-171.
//  - block scores: attn_gate.py:173-204 (q.k * scale, causal block mask, softmax), the
//    normalisation over key blocks of flashprefill_native_forward.py:365-374.
//  - selection: compact_attn/modules/flashprefill_prefill.py:596-666 and
//    compact_attn/modules/attention_forward_chunked_dense.py:352-403,559-638.
//  - union + compaction: attention_forward_chunked_dense.py:641-683,
//    compact_attn/kernels/varlen/flashinfer_zero_copy_prefill.py:482-510,
//    compact_attn/csrc/compactattn/cache_fill_kernel.cu:328-505.
//
// Every reduction that feeds a selection decision runs in a fixed order (see ca_common.h),
// so the scores and tables equal a sequential CPU evaluation bit for bit.

#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {
namespace {

// ---------------------------------------------------------------------------------------
// Gate projection (per head [in, 128], y[o] = sum_i x[i] W[i][o], sequential fma over
// i = 0 .. in-1) and block RoPE y[i] = x[i] cos[i] + rotate_half(x)[i] sin[i] (t1 = x cos,
// t2 = rot sin, y = t1 + t2).  128 threads per head: thread u owns output u; the weights of
// 32 inputs are loaded before their fmas (in is a multiple of 128), and the rotate_half
// partner of an output comes through ybuf ([128] floats of LDS).  Every thread of the
// workgroup calls this (it holds barriers); `active` threads compute.  Without w the input
// (in = 128) is rotated as it is.
__device__ void gate_project_rope(const float* xs, int in, const float* w, const float* rope_cos,
                                  const float* rope_sin, int64_t pos, float* out, int u, bool active,
                                  float* ybuf) {
    float a = 0.0f;
    if (active) {
        if (w == nullptr) a = xs[u];
        constexpr int kBatch = 32;
        for (int i0 = 0; w != nullptr && i0 < in; i0 += kBatch) {
            float wv[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) wv[j] = w[(i0 + j) * kD + u];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) a = __builtin_fmaf(xs[i0 + j], wv[j], a);
        }
    }
    if (rope_cos == nullptr) {
        if (active) out[u] = a;
        return;
    }
    if (active) ybuf[u] = a;
    __syncthreads();
    if (active) {
        const float rot = u < 64 ? -ybuf[u + 64] : ybuf[u - 64];
        const float t1 = a * rope_cos[pos * kD + u];
        const float t2 = rot * rope_sin[pos * kD + u];
        out[u] = t1 + t2;
    }
    __syncthreads();  // ybuf is free again
}

// ---------------------------------------------------------------------------------------
// Block staging shared by cache fill and query pooling: 256 threads move one 64-token x 128
// block with 16-byte accesses (thread t: token t/16 + 16 i, 8-element chunk t%16) and keep
// a bf16 copy in LDS; the block mean is then a sequential sum over the block's nv tokens per
// head dim (threads 0..127), divided by nv.  A chunk's last block holds nv < 64 tokens when
// its length is not a multiple of 64: only those rows are read, written and pooled.
constexpr int kTilePitch = kD + 8;  // bf16 elements per staged token row

// tokens of block j of a chunk of q_len tokens
__device__ __forceinline__ int block_tokens(int q_len, int j) {
    return min(kBlock, q_len - j * kBlock);
}

__device__ __forceinline__ float block_mean_from_lds(const uint16_t* tile, int d, int nv) {
    float sum = 0.0f;
#pragma unroll 16
    for (int t = 0; t < nv; ++t) sum = sum + bf16_to_f32(tile[t * kTilePitch + d]);
    return sum / static_cast<float>(nv);  // = sum * (1/64) bit for bit when nv = 64
}

// AttnGate pooling of head dim d over the nv staged tokens (attn_gate.py:113-130,233-237):
// the selected pools in the order max, min, avg go to xs[c*128 + d], c = 0, 1, ...  max and
// min are strict compares from token 0 (bf16 values, exact); avg is block_mean_from_lds.
__device__ __forceinline__ void block_pool_from_lds(const uint16_t* tile, int d, int pools, int nv, float* xs) {
    float mx = bf16_to_f32(tile[d]), mn = mx, sum = 0.0f;
#pragma unroll 16
    for (int t = 0; t < nv; ++t) {
        const float v = bf16_to_f32(tile[t * kTilePitch + d]);
        mx = v > mx ? v : mx;
        mn = v < mn ? v : mn;
        sum = sum + v;
    }
    int c = 0;
    if (pools & CA_POOL_MAX) xs[kD * c++ + d] = mx;
    if (pools & CA_POOL_MIN) xs[kD * c++ + d] = mn;
    if (pools & CA_POOL_AVG) xs[kD * c++ + d] = sum / static_cast<float>(nv);
}

__device__ __forceinline__ int pool_count(int pools) {
    return (pools & 1) + ((pools >> 1) & 1) + ((pools >> 2) & 1);
}

typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));

// Cache fill of new block j of (request x KV head) `row` by one workgroup of 256 threads;
// tile ([64][kTilePitch] bf16) and xs (3 * 128 floats) are its LDS.
__device__ __forceinline__ void cache_fill_block(const Shape& s, const SeqAddr& kn, const SeqAddr& vn,
                                                 const KvAddr& kc, const KvAddr& vc, const PastBlocks& pb,
                                                 float* kmean, const float* wk, const float* rope_cos,
                                                 const float* rope_sin, float* kgate, int pools, int gk, int j,
                                                 int row, uint16_t* tile, float* xs, float* ybuf) {
    const int b = row / s.Hkv;
    const int hk = row - b * s.Hkv;
    const int kb = pb.p[b] + j;
    const int nv = block_tokens(s.Lq, j);
    const int t = threadIdx.x;
    const int tok0 = t >> 4;
    const int ch = t & 15;
    const uint16_t* ks = kn.data + b * kn.sb + (int64_t)j * kBlock * kn.st + hk * kn.sh + 8 * ch;
    u32x4_v kr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32x4_v z = {0u, 0u, 0u, 0u};
        kr[i] = tok0 + 16 * i < nv ? *reinterpret_cast<const u32x4_v*>(ks + (int64_t)(tok0 + 16 * i) * kn.st) : z;
    }
    if (kc.data != nullptr) {  // append K and V (summaries-only calls pass no cache)
        const int64_t kphys = kc.page_table ? clamp_page(kc.page_table[(int64_t)row * kc.pts + kb], kc.max_page) : kb;
        const int64_t vphys = vc.page_table ? clamp_page(vc.page_table[(int64_t)row * vc.pts + kb], vc.max_page) : kb;
        const uint16_t* vsrc = vn.data + b * vn.sb + (int64_t)j * kBlock * vn.st + hk * vn.sh + 8 * ch;
        uint16_t* kd = kc.data + b * kc.sb + hk * kc.sh + kphys * kc.sblk + 8 * ch;
        uint16_t* vd = vc.data + b * vc.sb + hk * vc.sh + vphys * vc.sblk + 8 * ch;
        u32x4_v vr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4_v z = {0u, 0u, 0u, 0u};
            vr[i] = tok0 + 16 * i < nv ? *reinterpret_cast<const u32x4_v*>(vsrc + (int64_t)(tok0 + 16 * i) * vn.st) : z;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = tok0 + 16 * i;
            if (tok < nv) {
                *reinterpret_cast<u32x4_v*>(kd + (int64_t)tok * kc.stok) = kr[i];
                *reinterpret_cast<u32x4_v*>(vd + (int64_t)tok * vc.stok) = vr[i];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4_v*>(tile + (tok0 + 16 * i) * kTilePitch + 8 * ch) = kr[i];
    if (kmean == nullptr && wk == nullptr) return;
    __syncthreads();
    if (t < kD) {
        if (kmean) kmean[((int64_t)row * s.cap + kb) * kD + t] = block_mean_from_lds(tile, t, nv);
        if (wk) block_pool_from_lds(tile, t, pools, nv, xs);
    }
    if (wk == nullptr) return;
    __syncthreads();
    // gk gate heads per KV head: 1 (W_k per KV head) or G (the K block repeated to the Q heads
    // hk*G + j and projected per Q head, attn_gate.py:30-33,84-86); two heads at a time
    const int in = kD * pool_count(pools);
    for (int base = 0; base < gk; base += 2) {
        const int jh = base + (t >> 7);
        const bool active = jh < gk;
        const int64_t gh = (int64_t)row * gk + (active ? jh : 0);  // gate-head row (b*Hkv + hk)*gk + jh
        gate_project_rope(xs, in, wk + (int64_t)(hk * gk + (active ? jh : 0)) * in * kD, rope_cos, rope_sin, kb,
                          kgate + (gh * s.cap + kb) * kD, t & 127, active, ybuf + 128 * (t >> 7));
    }
}

// Cache fill: one (new block, request x KV head) per workgroup.
__global__ __launch_bounds__(256) void cache_fill_kernel(Shape s, SeqAddr kn, SeqAddr vn,
                                                         KvAddr kc, KvAddr vc, PastBlocks pb,
                                                         float* kmean, const float* wk,
                                                         const float* rope_cos,
                                                         const float* rope_sin, float* kgate, int pools,
                                                         int gk) {
    __shared__ __attribute__((aligned(16))) uint16_t tile[kBlock * kTilePitch];
    __shared__ float xs[3 * kD];
    __shared__ float ybuf[2 * kD];
    cache_fill_block(s, kn, vn, kc, vc, pb, kmean, wk, rope_cos, rope_sin, kgate, pools, gk, blockIdx.x, blockIdx.y,
                     tile, xs, ybuf);
}

// ---------------------------------------------------------------------------------------
// Query-block summaries: the AttnGate pools (or the FlashPrefill mean) of one 64-token block,
// optionally gate-projected and rotated.  One (block, request x head) per workgroup; with
// kv_aware one (block, request x KV head) per workgroup, whose G heads' pooled vectors are
// concatenated (g-major) before a per-KV-head projection (kv_group_aware_query,
// attn_gate.py:74-79,96-113).

// Summary of query block qb of (request x head) bh by one workgroup of 256 threads; xs holds
// the pooled vectors (nsrc * pools * 128 floats).
__device__ __forceinline__ void pool_query_block(const Shape& s, const SeqAddr& q, const PastBlocks& pb,
                                                 const float* wq, const float* rope_cos, const float* rope_sin,
                                                 float* qhat, int pools, int kv_aware, int qb, int bh,
                                                 uint16_t* tile, float* xs, float* ybuf) {
    const int heads = kv_aware ? s.Hkv : s.Hq;
    const int b = bh / heads;
    const int h = bh - b * heads;
    const int t = threadIdx.x;
    const int tok0 = t >> 4;
    const int ch = t & 15;
    const int C = pool_count(pools);
    const int nsrc = kv_aware ? s.G : 1;
    const int nv = block_tokens(s.Lq, qb);
    float* out = qhat + ((int64_t)bh * s.Qb + qb) * kD;
    for (int g = 0; g < nsrc; ++g) {
        const int hq = kv_aware ? h * s.G + g : h;
        const uint16_t* sp = q.data + b * q.sb + (int64_t)qb * kBlock * q.st + hq * q.sh + 8 * ch;
        if (g > 0) __syncthreads();  // the previous head's pooling is done with the tile
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = tok0 + 16 * i;
            if (tok < nv)
                *reinterpret_cast<u32x4_v*>(tile + tok * kTilePitch + 8 * ch) =
                    *reinterpret_cast<const u32x4_v*>(sp + (int64_t)tok * q.st);
        }
        __syncthreads();
        if (t < kD) {
            block_pool_from_lds(tile, t, pools, nv, xs + g * C * kD);
            if (wq == nullptr && rope_cos == nullptr) out[t] = xs[t];  // one pool, no projection, no RoPE
        }
    }
    if (wq == nullptr && rope_cos == nullptr) return;
    __syncthreads();
    const int in = nsrc * C * kD;
    const float* w = wq != nullptr ? wq + (int64_t)h * in * kD : nullptr;
    gate_project_rope(xs, in, w, rope_cos, rope_sin, (int64_t)pb.p[b] + qb, out, t & 127, t < 128, ybuf);
}

__global__ __launch_bounds__(256) void pool_query_kernel(Shape s, SeqAddr q, PastBlocks pb,
                                                         const float* wq, const float* rope_cos,
                                                         const float* rope_sin, float* qhat, int pools,
                                                         int kv_aware) {
    __shared__ __attribute__((aligned(16))) uint16_t tile[kBlock * kTilePitch];
    __shared__ float ybuf[kD];
    extern __shared__ float xs[];  // nsrc * pools * 128 pooled values (sized at launch)
    pool_query_block(s, q, pb, wq, rope_cos, rope_sin, qhat, pools, kv_aware, blockIdx.x, blockIdx.y, tile, xs,
                     ybuf);
}

// The chunk's FlashPrefill summaries in one launch: workgroup rows y < B*Hkv append the new
// K/V blocks and write their mean-K (cache_fill_kernel without a gate), the others pool the
// query blocks into their means (pool_query_kernel without a projection).
__global__ __launch_bounds__(256) void chunk_summaries_kernel(Shape s, SeqAddr kn, SeqAddr vn, KvAddr kc,
                                                              KvAddr vc, PastBlocks pb, float* kmean, SeqAddr q,
                                                              float* qhat) {
    __shared__ __attribute__((aligned(16))) uint16_t tile[kBlock * kTilePitch];
    __shared__ float xs[3 * kD];
    const int nkv = s.B * s.Hkv;
    if ((int)blockIdx.y < nkv)
        cache_fill_block(s, kn, vn, kc, vc, pb, kmean, nullptr, nullptr, nullptr, nullptr, CA_POOL_AVG, 1, blockIdx.x,
                         blockIdx.y, tile, xs, nullptr);
    else
        pool_query_block(s, q, pb, nullptr, nullptr, nullptr, qhat, CA_POOL_AVG, 0, blockIdx.x, blockIdx.y - nkv,
                         tile, xs, nullptr);
}

// ---------------------------------------------------------------------------------------
// Block logits: logits[(b*Hq + h)*Qb + qb][kb] = dot(qhat[b,h,qb], khat[b, h/G, kb]) * scale
// for the causal kb <= P + qb.  The G*Qb query vectors of a KV group are contiguous in
// qhat, so a workgroup takes a 64 (query vectors) x KT (key blocks) tile of one group;
// each thread owns a 4 x KT/16 register tile and every dot product is one sequential fma
// chain over d = 0..127.
constexpr int kPadRow = kD + 4;  // LDS row pitch (floats) for summary tiles
constexpr int kLogitsGridSlots = 512;  // block-logits workgroups resident at once (2 per CU)

// One workgroup computes a 64-row x KT-key tile of logits (KT = 32: twice the workgroups of
// 64-key tiles, so the last round of the grid carries half as much work per CU).  The first
// `extra` tiles of a row hold one key more (tile x starts at KT x + min(x, extra)): a row
// whose keys need just over a multiple of two workgroups per CU stays in one round of the
// grid instead of spilling a few tiles into a second (config 2: 2064 keys per row as 64
// tiles, 16 of them of 33 keys).  Wave 0 computes the extra key's 64 logits, one fma chain
// per row in the same order.
template <int KT>
__global__ __launch_bounds__(256) void block_logits_kernel(Shape s, const float* qhat, const float* khat,
                                                           float scale, PastBlocks pb, float* logits, int extra) {
    static_assert(KT == 32 || KT == 64, "16 key groups of KT/16 keys");
    constexpr int KJ = KT / 16;  // keys per thread
    __shared__ __attribute__((aligned(16))) float qt[64 * kPadRow];
    __shared__ __attribute__((aligned(16))) float kt[(KT + 1) * kPadRow];
    const int kb0 = blockIdx.x * KT + min((int)blockIdx.x, extra);
    const bool has_extra = (int)blockIdx.x < extra;
    const int row = blockIdx.y;
    const int m0 = blockIdx.z * 64;
    const int b = row / s.Hkv;
    const int hk = row - b * s.Hkv;
    const int P = pb.p[b];
    const int nkb = P + s.Qb;
    const int M = s.G * s.Qb;
    if (kb0 >= nkb || m0 >= M) return;
    const int t = threadIdx.x;
    const float* qbase = qhat + ((int64_t)(b * s.Hq + hk * s.G) * s.Qb + m0) * kD;
    const float* kbase = khat + ((int64_t)row * s.cap + kb0) * kD;
    const int mrows = min(64, M - m0);
    const int krows = min(KT + (has_extra ? 1 : 0), nkb - kb0);
    {
        // all loads of a thread in flight before the LDS stores
        constexpr int kQIters = 64 * (kD / 4) / 256;
        constexpr int kKIters = KT * (kD / 4) / 256;
        float4 qv[kQIters], kv[kKIters];
        // unconditional loads (rows past the tile's last valid row re-read that row; their
        // logits are computed and never stored), so all of them are in flight at once
#pragma unroll
        for (int i = 0; i < kQIters; ++i) {
            const int f = t + 256 * i;
            const int r = f >> 5, c4 = f & 31;
            qv[i] = *reinterpret_cast<const float4*>(qbase + (int64_t)min(r, mrows - 1) * kD + c4 * 4);
        }
#pragma unroll
        for (int i = 0; i < kKIters; ++i) {
            const int f = t + 256 * i;
            const int r = f >> 5, c4 = f & 31;
            kv[i] = *reinterpret_cast<const float4*>(kbase + (int64_t)min(r, krows - 1) * kD + c4 * 4);
        }
#pragma unroll
        for (int i = 0; i < kQIters; ++i) {
            const int f = t + 256 * i;
            const int r = f >> 5, c4 = f & 31;
            *reinterpret_cast<float4*>(qt + r * kPadRow + c4 * 4) = qv[i];
        }
#pragma unroll
        for (int i = 0; i < kKIters; ++i) {
            const int f = t + 256 * i;
            const int r = f >> 5, c4 = f & 31;
            *reinterpret_cast<float4*>(kt + r * kPadRow + c4 * 4) = kv[i];
        }
        if (has_extra && t < 32)  // key KT of the tile (re-read of the last valid row past nkb)
            *reinterpret_cast<float4*>(kt + KT * kPadRow + t * 4) =
                *reinterpret_cast<const float4*>(kbase + (int64_t)min(KT, krows - 1) * kD + t * 4);
    }
    __syncthreads();
    const int lane = t & 63;
    const int tm = lane & 15;              // query rows tm + 16 i
    const int tn = (t >> 6) * 4 + (lane >> 4);  // key rows KJ tn + j
    float acc[4][KJ];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < KJ; ++j) acc[i][j] = 0.0f;
    for (int d = 0; d < kD; d += 4) {
        float4 a[4], c[KJ];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const float4*>(qt + (tm + 16 * i) * kPadRow + d);
#pragma unroll
        for (int j = 0; j < KJ; ++j) c[j] = *reinterpret_cast<const float4*>(kt + (KJ * tn + j) * kPadRow + d);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < KJ; ++j) {
                float v = acc[i][j];
                v = __builtin_fmaf(a[i].x, c[j].x, v);
                v = __builtin_fmaf(a[i].y, c[j].y, v);
                v = __builtin_fmaf(a[i].z, c[j].z, v);
                v = __builtin_fmaf(a[i].w, c[j].w, v);
                acc[i][j] = v;
            }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + tm + 16 * i;
        if (m >= M) continue;
        const int qb = m % s.Qb;
        float* out = logits + ((int64_t)(b * s.Hq + hk * s.G) * s.Qb + m) * s.cap;
#pragma unroll
        for (int j = 0; j < KJ; ++j) {
            const int kb = kb0 + KJ * tn + j;
            if (kb <= P + qb) out[kb] = acc[i][j] * scale;
        }
    }
    if (has_extra && t < 64) {
        // key KT of the tile for query row t: the same sequential fma chain over d = 0..127
        // (after the tile: beside the tile's chains, in every wave, it measured slower)
        const int m = m0 + t;
        float v = 0.0f;
        for (int d = 0; d < kD; d += 4) {
            const float4 a = *reinterpret_cast<const float4*>(qt + t * kPadRow + d);
            const float4 c = *reinterpret_cast<const float4*>(kt + KT * kPadRow + d);
            v = __builtin_fmaf(a.x, c.x, v);
            v = __builtin_fmaf(a.y, c.y, v);
            v = __builtin_fmaf(a.z, c.z, v);
            v = __builtin_fmaf(a.w, c.w, v);
        }
        const int kb = kb0 + KT;
        if (m < M && kb <= P + m % s.Qb)
            logits[((int64_t)(b * s.Hq + hk * s.G) * s.Qb + m) * s.cap + kb] = v * scale;
    }
}

// ---------------------------------------------------------------------------------------
// Row softmax + selection, one workgroup per (b, h, qb) row.  Softmax sum order: lane l
// sums kb = l, l+64, ... ascending, then the tree part[l] += part[l+s], s = 32..1.
struct SelectParams {
    Shape s;
    float* scores;          // [B*Hq*Qb][cap]: logits in, probabilities out (compute mode)
    const void* scores_in;  // caller scores (select mode)
    int dtype;
    int64_t ssb, ssh, ssq;
    ca_select_rule rule;
    PastBlocks pb;
    uint32_t* rowmask;
};

// Monotone uint32 key of a float (larger float -> larger key); -0 is folded onto +0.
__device__ __forceinline__ uint32_t order_key(float v) {
    uint32_t u = __float_as_uint(v);
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ bool is_finite_f(float v) {
    return (__float_as_uint(v) & 0x7f800000u) != 0x7f800000u;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// The per-row selection runs one 256-thread workgroup per (b, h, qb) row; the row lives in
// LDS.  Top-k is exact on the order (score desc, block id asc):
//  1. a lower bound T_lo of the k-th largest key: the k-th largest of the 64 lane maxima
//     (at least k distinct keys are >= it), for k <= 64;
//  2. the keys >= T_lo (usually a few more than k) are gathered into a candidate list;
//  3. the k-th largest key T and the id cut among keys equal to T are found over the list
//     by bitwise construction with wave ballots.
// A list that overflows (heavy ties, k > 64) falls back to the same search over the row.
constexpr int kSelThreads = 256;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kCandSlots = 4;
constexpr int kCandCap = 64 * kCandSlots;

// Largest T with #{x >= T} >= k over the wave's S*64 values: the k-th largest (k >= 1).
template <int S>
__device__ __forceinline__ uint32_t wave_kth_largest(const uint32_t (&x)[S], int k) {
    uint32_t T = 0;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t c = T | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < S; ++i) cnt += __popcll(__ballot(x[i] >= c));
        if (cnt >= k) T = c;
    }
    return T;
}

// Largest T with #{sel && id < T} < k over ids < 2^16: the k-th smallest selected id.
template <int S>
__device__ __forceinline__ int wave_kth_smallest_id(const int (&id)[S], const bool (&sel)[S], int k) {
    int T = 0;
    for (int bit = 15; bit >= 0; --bit) {
        const int c = T | (1 << bit);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < S; ++i) cnt += __popcll(__ballot(sel[i] && id[i] < c));
        if (cnt < k) T = c;
    }
    return T;
}

// The k-th largest key T over the nl (<= 64 S) candidates held S per lane, and the id cut
// among the candidates equal to T: the (k - #{key > T})-th smallest such id.
template <int S>
__device__ __forceinline__ void select_candidates(const uint32_t* cand_key, const int* cand_id, int nl, int lane,
                                                  int k, uint32_t& T, int& eq_cut) {
    uint32_t x[S];
    int id[S];
    bool eq[S];
#pragma unroll
    for (int i = 0; i < S; ++i) {
        const int j = lane + 64 * i;
        x[i] = j < nl ? cand_key[j] : 0u;
        id[i] = j < nl ? cand_id[j] : 0;
    }
    T = wave_kth_largest<S>(x, k);
    int gt = 0;
#pragma unroll
    for (int i = 0; i < S; ++i) {
        gt += __popcll(__ballot(x[i] > T));
        eq[i] = x[i] == T;
    }
    eq_cut = wave_kth_smallest_id<S>(id, eq, k - gt);
}

template <bool kCompute>
__global__ __launch_bounds__(kSelThreads) void row_select_kernel(SelectParams p) {
    extern __shared__ float row[];  // [cap]
    __shared__ float red_f[kSelWaves];
    __shared__ int red_i[kSelWaves];
    __shared__ int red_z[kSelWaves];
    __shared__ uint32_t tmax[kSelThreads];
    __shared__ uint32_t cand_key[kCandCap];
    __shared__ int cand_id[kCandCap];
    __shared__ int cand_n;
    __shared__ uint32_t sel_lo, sel_T;
    __shared__ int sel_cut;
    const Shape& s = p.s;
    const int rid = blockIdx.x;  // (b*Hq + h)*Qb + qb
    const int qb = rid % s.Qb;
    const int bh = rid / s.Qb;
    const int b = bh / s.Hq;
    const int h = bh - b * s.Hq;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int P = p.pb.p[b];
    const int qabs = P + qb;
    const int n = qabs + 1;
    const int cap = s.cap;
    constexpr float kNegInf = -__builtin_inff();

    if (kCompute) {
        float* srow = p.scores + (int64_t)rid * cap;
        float m = kNegInf;
        for (int base = 0; base < n; base += 4 * kSelThreads) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kb = base + t + kSelThreads * i;
                v[i] = kb < n ? srow[kb] : kNegInf;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kb = base + t + kSelThreads * i;
                if (kb < n) row[kb] = v[i];
                m = fmaxf(m, v[i]);
            }
        }
        m = wave_max(m);
        if (lane == 0) red_f[wave] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
        for (int kb = t; kb < n; kb += kSelThreads) row[kb] = exp_fixed(row[kb] - m);
        __syncthreads();
        if (wave == 0) {
            // lane l sums kb = l, l + 64, ... in ascending order, then the fixed tree
            float part = 0.0f;
            for (int base = 0; base < n; base += 8 * 64) {
                float e[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int kb = base + lane + 64 * i;
                    e[i] = kb < n ? row[kb] : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (base + lane + 64 * i < n) part = part + e[i];
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) part = part + __shfl_down(part, o, 64);
            if (lane == 0) red_f[0] = part;
        }
        __syncthreads();
        const float sum = red_f[0];
        for (int kb = t; kb < cap; kb += kSelThreads) {
            float v = 0.0f;
            if (kb < n) {
                v = row[kb] / sum;
                row[kb] = v;
            }
            srow[kb] = v;
        }
    } else {
        const int64_t off = b * p.ssb + h * p.ssh + qb * p.ssq;
        for (int base = 0; base < n; base += 4 * kSelThreads) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kb = base + t + kSelThreads * i;
                v[i] = 0.0f;
                if (kb < n) {
                    if (p.dtype == 0)
                        v[i] = static_cast<const float*>(p.scores_in)[off + kb];
                    else
                        v[i] = bf16_to_f32(static_cast<const uint16_t*>(p.scores_in)[off + kb]);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kb = base + t + kSelThreads * i;
                if (kb < n) row[kb] = v[i];
            }
        }
    }
    __syncthreads();

    // Row statistics: the alpha rule's row max, the top-k candidate count and the
    // per-thread maximum candidate key (top-k bound).
    //  - Row max: the max over all Kb = P + Qb columns of the zeroed row, where non-causal
    //    and non-finite entries read as 0 (flashprefill_prefill.py:633-645).
    //  - Top-k candidates: the finite past blocks kb < P (past-only form), or every column
    //    kb < Kb with its zeroed value (CA_RULE_TOPK_ALLCOLS, the reference's min_budget:
    //    torch.topk over the zeroed row, :637-643); picks past the causal edge are dropped.
    const ca_select_rule& rule = p.rule;
    const int Kb = P + s.Qb;
    const bool all_cols = (rule.flags & CA_RULE_TOPK_ALLCOLS) != 0;
    const int kend = all_cols ? Kb : P;
    const bool use_topk = (rule.flags & CA_RULE_TOPK) && rule.topk > 0 && kend > 0;
    auto cand_val = [&](int kb, float& v) -> bool {
        if (all_cols) {
            v = kb < n ? row[kb] : 0.0f;
            if (!is_finite_f(v)) v = 0.0f;
            return true;
        }
        v = row[kb];
        return is_finite_f(v);
    };
    {
        float mx = kNegInf;
        int nc = 0, nz = 0;
        uint32_t kmax = 0;
        const int lim = max(n, use_topk ? kend : 0);
        for (int kb = t; kb < lim; kb += kSelThreads) {
            if (kb < n) {
                const float v = row[kb];
                if (is_finite_f(v))
                    mx = fmaxf(mx, v);
                else
                    ++nz;
            }
            float cv;
            if (use_topk && kb < kend && cand_val(kb, cv)) {
                ++nc;
                kmax = max(kmax, order_key(cv));
            }
        }
        mx = wave_max(mx);
        nc = wave_sum_int(nc);
        nz = wave_sum_int(nz);
        tmax[t] = kmax;
        if (lane == 0) {
            red_f[wave] = mx;
            red_i[wave] = nc;
            red_z[wave] = nz;
        }
        if (t == 0) cand_n = 0;
    }
    __syncthreads();
    float rowmax = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
    if (n < Kb || red_z[0] + red_z[1] + red_z[2] + red_z[3] > 0) rowmax = fmaxf(rowmax, 0.0f);
    const int ncand = red_i[0] + red_i[1] + red_i[2] + red_i[3];
    const float alpha_cut = rule.alpha * rowmax;
    const bool take_all = use_topk && rule.topk >= ncand;
    const bool cut = use_topk && !take_all;
    const int k = rule.topk;

    if (cut) {
        if (wave == 0) {
            uint32_t lo = 0;
            if (k <= 64) {
                const uint32_t m[1] = {max(max(tmax[lane], tmax[lane + 64]),
                                           max(tmax[lane + 128], tmax[lane + 192]))};
                lo = wave_kth_largest<1>(m, k);
            }
            if (lane == 0) sel_lo = lo;
        }
        __syncthreads();
        const uint32_t lo = sel_lo;
        for (int kb = t; kb < kend; kb += kSelThreads) {
            float v;
            if (!cand_val(kb, v)) continue;
            const uint32_t key = order_key(v);
            if (key < lo) continue;
            const int slot = atomicAdd(&cand_n, 1);
            if (slot < kCandCap) {
                cand_key[slot] = key;
                cand_id[slot] = kb;
            }
        }
        __syncthreads();
        if (wave == 0) {
            const int nl = cand_n;
            uint32_t T;
            int eq_cut;
            if (nl <= 64) {
                // the usual case: one candidate per lane
                select_candidates<1>(cand_key, cand_id, nl, lane, k, T, eq_cut);
            } else if (nl <= kCandCap) {
                select_candidates<kCandSlots>(cand_key, cand_id, nl, lane, k, T, eq_cut);
            } else {
                T = 0;
                for (int bit = 31; bit >= 0; --bit) {
                    const uint32_t c = T | (1u << bit);
                    int cnt = 0;
                    for (int kb = lane; kb < kend; kb += 64) {
                        float v;
                        cnt += (cand_val(kb, v) && order_key(v) >= c) ? 1 : 0;
                    }
                    if (wave_sum_int(cnt) >= k) T = c;
                }
                int gt = 0;
                for (int kb = lane; kb < kend; kb += 64) {
                    float v;
                    gt += (cand_val(kb, v) && order_key(v) > T) ? 1 : 0;
                }
                const int krem = k - wave_sum_int(gt);
                // the krem-th key equal to T in ascending block order
                const uint64_t lt_mask = (1ull << lane) - 1ull;
                int seen = 0;
                eq_cut = kend;
                for (int base = 0; base < kend; base += 64) {
                    const int kb = base + lane;
                    float v = 0.0f;
                    const bool e = kb < kend && cand_val(kb, v) && order_key(v) == T;
                    const uint64_t bal = __ballot(e);
                    const int cnt = __popcll(bal);
                    if (seen + cnt >= krem) {
                        const uint64_t who = __ballot(e && seen + __popcll(bal & lt_mask) == krem - 1);
                        eq_cut = base + __ffsll(static_cast<unsigned long long>(who)) - 1;
                        break;
                    }
                    seen += cnt;
                }
            }
            if (lane == 0) {
                sel_T = T;
                sel_cut = eq_cut;
            }
        }
        __syncthreads();
    }
    const uint32_t T = cut ? sel_T : 0u;
    const int eq_cut = cut ? sel_cut : -1;

    uint32_t* out = p.rowmask + (int64_t)rid * s.words;
    const int chunks = (s.words + 1) / 2;
    for (int c = wave; c < chunks; c += kSelWaves) {
        const int kb = c * 64 + lane;
        bool keep = false;
        if (kb < n) {
            const float v = row[kb];
            const bool fin = is_finite_f(v);
            if ((rule.flags & CA_RULE_ALPHA) && fin && v >= alpha_cut) keep = true;
            if ((rule.flags & CA_RULE_THRESHOLD) && v > rule.threshold) keep = true;
            if (kb < rule.sink_blocks) keep = true;
            if (qabs - kb < rule.window_blocks) keep = true;
            if (kb < P && kb >= P - rule.local_blocks) keep = true;
            float cv;
            if (use_topk && kb < kend && cand_val(kb, cv)) {
                if (take_all) {
                    keep = true;
                } else {
                    const uint32_t key = order_key(cv);
                    if (key > T || (key == T && kb <= eq_cut)) keep = true;
                }
            }
        }
        const uint64_t bal = __ballot(keep);
        if (lane == 0) out[2 * c] = static_cast<uint32_t>(bal);
        if (lane == 1 && 2 * c + 1 < s.words) out[2 * c + 1] = static_cast<uint32_t>(bal >> 32);
    }
}

// The same row selection with the row held in registers, for rows of at most 256 * NR
// blocks: thread t owns blocks kb = t + 256 i (i < NR), which is also lane (kb % 64) of
// wave (kb / 64) % 4 in mask chunk kb / 64, so the masks come straight from registers.
//  - one round of global loads for the whole row;
//  - the softmax sum keeps the order above (wave 0 over the exponentials staged in LDS);
//  - every wave derives the top-k bound and the final cut itself from the shared lane
//    maxima and candidate list, which saves the broadcast barriers;
//  - the row is also staged in LDS for the whole-row search when the candidate list
//    overflows.
// Results are bit-identical to row_select_kernel.
template <bool kCompute, int NR>
__global__ __launch_bounds__(kSelThreads) void row_select_reg_kernel(SelectParams p) {
    extern __shared__ float row[];  // [cap]
    __shared__ float red_f[kSelWaves];
    __shared__ float red_sum;  // its own slot: the statistics below reuse red_f without a barrier
    __shared__ int red_i[kSelWaves];
    __shared__ int red_z[kSelWaves];
    __shared__ uint32_t tmax[kSelThreads];
    __shared__ uint32_t cand_key[kCandCap];
    __shared__ int cand_id[kCandCap];
    __shared__ int cand_n;
    __shared__ uint32_t sel_T;
    __shared__ int sel_cut;
    const Shape& s = p.s;
    const int rid = blockIdx.x;  // (b*Hq + h)*Qb + qb
    const int qb = rid % s.Qb;
    const int bh = rid / s.Qb;
    const int b = bh / s.Hq;
    const int h = bh - b * s.Hq;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int P = p.pb.p[b];
    const int qabs = P + qb;
    const int n = qabs + 1;
    const int cap = s.cap;
    constexpr float kNegInf = -__builtin_inff();

    float v[NR];  // logits, then probabilities (compute mode); caller scores (select mode)
    if (kCompute) {
        float* srow = p.scores + (int64_t)rid * cap;
        // unconditional loads of a clamped column (n >= 1), all in flight at once
#pragma unroll
        for (int i = 0; i < NR; ++i) v[i] = srow[min(t + kSelThreads * i, n - 1)];
#pragma unroll
        for (int i = 0; i < NR; ++i)
            if (t + kSelThreads * i >= n) v[i] = kNegInf;
        float m = kNegInf;
#pragma unroll
        for (int i = 0; i < NR; ++i) m = fmaxf(m, v[i]);
        m = wave_max(m);
        if (lane == 0) red_f[wave] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int kb = t + kSelThreads * i;
            if (kb < n) {
                v[i] = exp_fixed(v[i] - m);
                row[kb] = v[i];
            }
        }
        __syncthreads();
        if (wave == 0) {
            // lane l sums kb = l, l + 64, ... in ascending order, then the fixed tree
            float part = 0.0f;
            for (int base = 0; base < n; base += 8 * 64) {
                float e[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int kb = base + lane + 64 * i;
                    e[i] = kb < n ? row[kb] : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (base + lane + 64 * i < n) part = part + e[i];
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) part = part + __shfl_down(part, o, 64);
            if (lane == 0) red_sum = part;
        }
        __syncthreads();
        const float sum = red_sum;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int kb = t + kSelThreads * i;
            float pv = 0.0f;
            if (kb < n) {
                pv = v[i] / sum;
                row[kb] = pv;
            }
            v[i] = pv;
            if (kb < cap) srow[kb] = pv;
        }
    } else {
        const int64_t off = b * p.ssb + h * p.ssh + qb * p.ssq;
        // unconditional loads of a clamped column (n >= 1), all in flight at once
        if (p.dtype == 0) {
            const float* in = static_cast<const float*>(p.scores_in) + off;
#pragma unroll
            for (int i = 0; i < NR; ++i) v[i] = in[min(t + kSelThreads * i, n - 1)];
        } else {
            const uint16_t* in = static_cast<const uint16_t*>(p.scores_in) + off;
#pragma unroll
            for (int i = 0; i < NR; ++i) v[i] = bf16_to_f32(in[min(t + kSelThreads * i, n - 1)]);
        }
#pragma unroll
        for (int i = 0; i < NR; ++i)
            if (t + kSelThreads * i >= n) v[i] = 0.0f;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int kb = t + kSelThreads * i;
            if (kb < n) row[kb] = v[i];
        }
    }

    // Row statistics as in row_select_kernel: the zeroed row's max over all Kb columns,
    // the top-k candidate count and each thread's largest candidate key.
    const ca_select_rule& rule = p.rule;
    const int Kb = P + s.Qb;
    const bool all_cols = (rule.flags & CA_RULE_TOPK_ALLCOLS) != 0;
    const int kend = all_cols ? Kb : P;
    const bool use_topk = (rule.flags & CA_RULE_TOPK) && rule.topk > 0 && kend > 0;
    // candidate value of register i (block kb): the zeroed value over all columns, or a
    // finite past score
    auto cand_val = [&](int i, int kb, float& cv) -> bool {
        if (all_cols) {
            cv = kb < n ? v[i] : 0.0f;
            if (!is_finite_f(cv)) cv = 0.0f;
            return true;
        }
        cv = v[i];
        return is_finite_f(cv);
    };
    {
        float mx = kNegInf;
        int nc = 0, nz = 0;
        uint32_t kmax = 0;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int kb = t + kSelThreads * i;
            if (kb < n) {
                if (is_finite_f(v[i]))
                    mx = fmaxf(mx, v[i]);
                else
                    ++nz;
            }
            float cv;
            if (use_topk && kb < kend && cand_val(i, kb, cv)) {
                ++nc;
                kmax = max(kmax, order_key(cv));
            }
        }
        mx = wave_max(mx);
        nc = wave_sum_int(nc);
        nz = wave_sum_int(nz);
        tmax[t] = kmax;
        if (lane == 0) {
            red_f[wave] = mx;
            red_i[wave] = nc;
            red_z[wave] = nz;
        }
        if (t == 0) cand_n = 0;
    }
    __syncthreads();
    float rowmax = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
    if (n < Kb || red_z[0] + red_z[1] + red_z[2] + red_z[3] > 0) rowmax = fmaxf(rowmax, 0.0f);
    const int ncand = red_i[0] + red_i[1] + red_i[2] + red_i[3];
    const float alpha_cut = rule.alpha * rowmax;
    const bool take_all = use_topk && rule.topk >= ncand;
    const bool cut = use_topk && !take_all;
    const int k = rule.topk;

    uint32_t T = 0u;
    int eq_cut = -1;
    if (cut) {
        // every wave computes the same lower bound from the 64 lane maxima
        uint32_t lo = 0;
        if (k <= 64) {
            const uint32_t m1[1] = {max(max(tmax[lane], tmax[lane + 64]), max(tmax[lane + 128], tmax[lane + 192]))};
            lo = wave_kth_largest<1>(m1, k);
        }
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int kb = t + kSelThreads * i;
            float cv;
            if (kb < kend && cand_val(i, kb, cv)) {
                const uint32_t key = order_key(cv);
                if (key >= lo) {
                    const int slot = atomicAdd(&cand_n, 1);
                    if (slot < kCandCap) {
                        cand_key[slot] = key;
                        cand_id[slot] = kb;
                    }
                }
            }
        }
        __syncthreads();
        const int nl = cand_n;
        if (nl <= 64) {
            select_candidates<1>(cand_key, cand_id, nl, lane, k, T, eq_cut);  // every wave, same result
        } else if (nl <= kCandCap) {
            select_candidates<kCandSlots>(cand_key, cand_id, nl, lane, k, T, eq_cut);
        } else {
            // heavy ties or k > 64: wave 0 searches the staged row, as row_select_kernel does
            if (wave == 0) {
                auto row_val = [&](int kb, float& cv) -> bool {
                    if (all_cols) {
                        cv = kb < n ? row[kb] : 0.0f;
                        if (!is_finite_f(cv)) cv = 0.0f;
                        return true;
                    }
                    cv = row[kb];
                    return is_finite_f(cv);
                };
                uint32_t Tw = 0;
                for (int bit = 31; bit >= 0; --bit) {
                    const uint32_t c = Tw | (1u << bit);
                    int cnt = 0;
                    for (int kb = lane; kb < kend; kb += 64) {
                        float cv;
                        cnt += (row_val(kb, cv) && order_key(cv) >= c) ? 1 : 0;
                    }
                    if (wave_sum_int(cnt) >= k) Tw = c;
                }
                int gt = 0;
                for (int kb = lane; kb < kend; kb += 64) {
                    float cv;
                    gt += (row_val(kb, cv) && order_key(cv) > Tw) ? 1 : 0;
                }
                const int krem = k - wave_sum_int(gt);
                const uint64_t lt_mask = (1ull << lane) - 1ull;
                int seen = 0;
                int cutw = kend;
                for (int base = 0; base < kend; base += 64) {
                    const int kb = base + lane;
                    float cv = 0.0f;
                    const bool e = kb < kend && row_val(kb, cv) && order_key(cv) == Tw;
                    const uint64_t bal = __ballot(e);
                    const int cnt = __popcll(bal);
                    if (seen + cnt >= krem) {
                        const uint64_t who = __ballot(e && seen + __popcll(bal & lt_mask) == krem - 1);
                        cutw = base + __ffsll(static_cast<unsigned long long>(who)) - 1;
                        break;
                    }
                    seen += cnt;
                }
                if (lane == 0) {
                    sel_T = Tw;
                    sel_cut = cutw;
                }
            }
            __syncthreads();
            T = sel_T;
            eq_cut = sel_cut;
        }
    }

    // masks: register i of this thread is lane `lane` of chunk c = wave + 4 i
    uint32_t* out = p.rowmask + (int64_t)rid * s.words;
    const int chunks = (s.words + 1) / 2;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int c = wave + kSelWaves * i;
        if (c >= chunks) break;
        const int kb = c * 64 + lane;
        bool keep = false;
        if (kb < n) {
            const float x = v[i];
            const bool fin = is_finite_f(x);
            if ((rule.flags & CA_RULE_ALPHA) && fin && x >= alpha_cut) keep = true;
            if ((rule.flags & CA_RULE_THRESHOLD) && x > rule.threshold) keep = true;
            if (kb < rule.sink_blocks) keep = true;
            if (qabs - kb < rule.window_blocks) keep = true;
            if (kb < P && kb >= P - rule.local_blocks) keep = true;
            float cv;
            if (use_topk && kb < kend && cand_val(i, kb, cv)) {
                if (take_all) {
                    keep = true;
                } else {
                    const uint32_t key = order_key(cv);
                    if (key > T || (key == T && kb <= eq_cut)) keep = true;
                }
            }
        }
        const uint64_t bal = __ballot(keep);
        if (lane == 0) out[2 * c] = static_cast<uint32_t>(bal);
        if (lane == 1 && 2 * c + 1 < s.words) out[2 * c + 1] = static_cast<uint32_t>(bal >> 32);
    }
}

// ---------------------------------------------------------------------------------------
// Block-Union + compaction, one (request, KV head) row per workgroup of 256 threads.
struct UnionParams {
    Shape s;
    const uint32_t* rowmask;  // per-row masks (mode 0)
    const uint8_t* keep_kv_in;  // caller keep mask (mode 1)
    int mode;                   // 0: rowmask, 1: keep_kv_in, 2: dense
    int pooled;                 // query blocks taking part in the union
    PastBlocks pb;
    uint8_t* keep_block;
    uint8_t* keep_kv;
    int32_t* table;
    int64_t table_stride;
    int32_t* counts;
};

__device__ __forceinline__ uint32_t range_bits(int w, int lo, int hi) {
    // bits of word w for ids in [lo, hi)
    const int a = max(lo - 32 * w, 0);
    const int e = min(hi - 32 * w, 32);
    if (e <= a) return 0u;
    const uint32_t upper = e >= 32 ? 0xffffffffu : ((1u << e) - 1u);
    const uint32_t lower = (1u << a) - 1u;
    return upper & ~lower;
}

__global__ __launch_bounds__(256) void union_compact_kernel(UnionParams p) {
    extern __shared__ uint32_t lds_words[];  // [G][words] per-head union, then [words] KV union
    __shared__ int ired[8];
    const Shape& s = p.s;
    const int row = blockIdx.x;
    const int b = row / s.Hkv;
    const int hk = row - b * s.Hkv;
    const int t = threadIdx.x;
    const int P = p.pb.p[b];
    const int nkb = P + s.Qb;
    const int G = s.G;
    const int W = s.words;
    uint32_t* hw = lds_words;           // [G][W]
    uint32_t* kvw = lds_words + G * W;  // [W]
    if (p.mode == 0) {
        // thread i owns word w of head g: the OR over the pooled query blocks of the group's
        // row masks, eight independent loads in flight per batch
        const uint32_t* rm = p.rowmask + (int64_t)(b * s.Hq + hk * G) * s.Qb * W;
        for (int i = t; i < G * W; i += 256) {
            const int g = i / W;
            const int w = i - g * W;
            const uint32_t* src = rm + (int64_t)g * s.Qb * W + w;
            uint32_t acc = 0;
            int qb = 0;
            for (; qb + 8 <= p.pooled; qb += 8) {
                uint32_t v[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = src[(int64_t)(qb + k) * W];
#pragma unroll
                for (int k = 0; k < 8; ++k) acc |= v[k];
            }
            for (; qb < p.pooled; ++qb) acc |= src[(int64_t)qb * W];
            hw[i] = acc;
        }
        __syncthreads();
    }
    for (int w = t; w < W; w += 256) {
        const uint32_t valid = range_bits(w, 0, nkb);
        const uint32_t cur = range_bits(w, P, nkb);
        uint32_t acc = 0;
        if (p.mode == 0) {
            for (int g = 0; g < G; ++g) {
                const uint32_t x = (hw[g * W + w] | cur) & valid;
                if (p.keep_block) {
                    uint8_t* kbk = p.keep_block + ((int64_t)b * s.Hq + hk * G + g) * s.cap + 32 * w;
                    for (int i = 0; i < 32 && 32 * w + i < s.cap; ++i) kbk[i] = (x >> i) & 1u;
                }
                acc |= x;
            }
        } else if (p.mode == 1) {
            const uint8_t* src = p.keep_kv_in + (int64_t)row * s.cap + 32 * w;
            for (int i = 0; i < 32 && 32 * w + i < s.cap; ++i) acc |= (src[i] != 0 ? 1u : 0u) << i;
            acc = (acc | cur) & valid;
        } else {
            acc = valid;
        }
        if (p.keep_kv) {
            uint8_t* kv = p.keep_kv + (int64_t)row * s.cap + 32 * w;
            for (int i = 0; i < 32 && 32 * w + i < s.cap; ++i) kv[i] = (acc >> i) & 1u;
        }
        kvw[w] = acc;
    }
    __syncthreads();
    const int wpt = (W + 255) / 256;
    const int w0 = t * wpt;
    const int w1 = min(w0 + wpt, W);
    int cnt = 0;
    for (int w = w0; w < w1; ++w) cnt += __popc(kvw[w]);
    int total;
    int pos = block_exclusive_scan256(cnt, ired, &total);
    int32_t* tab = p.table + (int64_t)row * p.table_stride;
    for (int w = w0; w < w1; ++w) {
        uint32_t bits = kvw[w];
        while (bits) {
            const int i = __ffs(bits) - 1;
            tab[pos++] = 32 * w + i;
            bits &= bits - 1u;
        }
    }
    for (int i = total + t; i < s.cap; i += 256) tab[i] = -1;
    if (t == 0) p.counts[row] = total;
}

// ---------------------------------------------------------------------------------------
// Block tables -> CSR page lists (FlashInfer's paged-KV form): kv_indptr[r] is the exclusive
// prefix sum of the row counts, kv_indices[kv_indptr[r] + i] = r * kv_cap + table[r][i] (the
// global page id of the heads-first cache), kv_last_page_len[r] = 64.  One workgroup: the
// rows are scanned 1024 at a time, then each wave copies whole rows.
struct CsrParams {
    const int32_t* table;
    int64_t table_stride;
    const int32_t* counts;
    int rows;
    int cap;
    int32_t* indptr;
    int32_t* indices;
    int32_t* last_page_len;
};

constexpr int kCsrThreads = 1024;
constexpr int kCsrMaxRows = 8192;

__global__ __launch_bounds__(kCsrThreads) void table_csr_kernel(CsrParams p) {
    __shared__ int32_t off[kCsrMaxRows + 1];
    __shared__ int32_t wsum[kCsrThreads / 64];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wv = t >> 6;
    int carry = 0;
    for (int base = 0; base < p.rows; base += kCsrThreads) {
        const int r = base + t;
        const int c = r < p.rows ? min(max(p.counts[r], 0), p.cap) : 0;
        // inclusive scan inside the wave
        int x = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        if (lane == 63) wsum[wv] = x;
        __syncthreads();
        int before = carry;
        for (int v = 0; v < wv; ++v) before += wsum[v];
        int total = carry;
        for (int v = 0; v < kCsrThreads / 64; ++v) total += wsum[v];
        if (r < p.rows) off[r] = before + x - c;
        __syncthreads();  // wsum is rewritten by the next chunk
        carry = total;
    }
    if (t == 0) off[p.rows] = carry;
    __syncthreads();
    for (int r = t; r <= p.rows; r += kCsrThreads) p.indptr[r] = off[r];
    if (p.last_page_len)
        for (int r = t; r < p.rows; r += kCsrThreads) p.last_page_len[r] = 64;
    for (int r = wv; r < p.rows; r += kCsrThreads / 64) {
        const int c = off[r + 1] - off[r];
        const int32_t* src = p.table + (int64_t)r * p.table_stride;
        int32_t* dst = p.indices + off[r];
        const int gbase = r * p.cap;
        for (int i = lane; i < c; i += 64) dst[i] = gbase + min(max(src[i], 0), p.cap - 1);
    }
}


// 128-token block summaries from pairs of 64-token ones (FlashPrefill with 128-token score
// blocks): dst[j] = (c0 * src[2j] + c1 * src[2j + 1]) / (c0 + c1) with the blocks' token counts
// c (64, or last_tokens for the last source block) -- two products, one sum, one correctly
// rounded division, in that order -- and dst[j] = src[2j] when block 2j has no partner.  One
// thread per four head dims of one (row, pair).
__global__ __launch_bounds__(256) void pair_summaries_kernel(const float* src, int64_t src_stride, float* dst,
                                                             int64_t dst_stride, int64_t rows, int n_blocks,
                                                             int last_tokens) {
    const int npairs = (n_blocks + 1) / 2;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= rows * npairs * 32) return;
    const int q = static_cast<int>(gid & 31);
    const int64_t rp = gid >> 5;
    const int64_t row = rp / npairs;
    const int j = static_cast<int>(rp - row * npairs);
    const int b0 = 2 * j;
    const float* s0 = src + (row * src_stride + b0) * kD + 4 * q;
    float4 out = *reinterpret_cast<const float4*>(s0);
    if (b0 + 1 < n_blocks) {
        const float c0 = b0 == n_blocks - 1 ? static_cast<float>(last_tokens) : 64.0f;
        const float c1 = b0 + 1 == n_blocks - 1 ? static_cast<float>(last_tokens) : 64.0f;
        const float4 m1 = *reinterpret_cast<const float4*>(s0 + kD);
        const float n = c0 + c1;
        const float4 m0 = out;
        out.x = (c0 * m0.x + c1 * m1.x) / n;
        out.y = (c0 * m0.y + c1 * m1.y) / n;
        out.z = (c0 * m0.z + c1 * m1.z) / n;
        out.w = (c0 * m0.w + c1 * m1.w) / n;
    }
    *reinterpret_cast<float4*>(dst + (row * dst_stride + j) * kD + 4 * q) = out;
}

}  // namespace

hipError_t launch_cache_fill(const Shape& s, const SeqAddr& k_new, const SeqAddr& v_new,
                             const KvAddr& k_cache, const KvAddr& v_cache, const PastBlocks& pb,
                             float* kmean, const float* wk, const float* rope_cos,
                             const float* rope_sin, float* kgate, int pools, int gk, hipStream_t stream) {
    dim3 grid(s.Qb, s.B * s.Hkv);
    hipLaunchKernelGGL(cache_fill_kernel, grid, dim3(256), 0, stream, s, k_new, v_new, k_cache,
                       v_cache, pb, kmean, wk, rope_cos, rope_sin, kgate, pools, gk);
    return hipGetLastError();
}

hipError_t launch_chunk_summaries(const Shape& s, const SeqAddr& k_new, const SeqAddr& v_new, const KvAddr& k_cache,
                                  const KvAddr& v_cache, const PastBlocks& pb, float* kmean, const SeqAddr& q,
                                  float* qhat, hipStream_t stream) {
    dim3 grid(s.Qb, s.B * (s.Hkv + s.Hq));
    hipLaunchKernelGGL(chunk_summaries_kernel, grid, dim3(256), 0, stream, s, k_new, v_new, k_cache, v_cache, pb,
                       kmean, q, qhat);
    return hipGetLastError();
}

hipError_t launch_pool_query(const Shape& s, const SeqAddr& q, const PastBlocks& pb, const float* wq,
                             const float* rope_cos, const float* rope_sin, float* qhat, int pools,
                             bool kv_aware, hipStream_t stream) {
    dim3 grid(s.Qb, s.B * (kv_aware ? s.Hkv : s.Hq));
    // the pooled vectors of one output: G heads (kv-aware) or one, times the pools
    const size_t xs_bytes = sizeof(float) * kD * (kv_aware ? s.G : 1) * __builtin_popcount(pools & 7);
    hipLaunchKernelGGL(pool_query_kernel, grid, dim3(256), xs_bytes, stream, s, q, pb, wq, rope_cos,
                       rope_sin, qhat, pools, kv_aware ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_pair_summaries(const float* src, int64_t src_stride, float* dst, int64_t dst_stride,
                                 int64_t rows, int n_blocks, int last_tokens, hipStream_t stream) {
    const int64_t threads = rows * ((n_blocks + 1) / 2) * 32;
    hipLaunchKernelGGL(pair_summaries_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0,
                       stream, src, src_stride, dst, dst_stride, rows, n_blocks, last_tokens);
    return hipGetLastError();
}

size_t score_select_lds_bytes(const Shape& s, bool compute) {
    (void)compute;
    return sizeof(float) * (size_t)s.cap;
}

hipError_t launch_score_select(const Shape& s, const float* qhat, const float* khat, float scale,
                               const void* scores_in, int dtype, int64_t ssb, int64_t ssh,
                               int64_t ssq, const ca_select_rule& rule, const PastBlocks& pb,
                               uint32_t* rowmask, float* scores, hipStream_t stream) {
    const bool compute = scores_in == nullptr;
    if (compute) {
        int max_nkb = 0;
        for (int b = 0; b < s.B; ++b) max_nkb = max(max_nkb, pb.p[b] + s.Qb);
        constexpr int kKT = 32;
        const int rows_z = s.B * s.Hkv * ((s.G * s.Qb + 63) / 64);
        int tiles = (max_nkb + kKT - 1) / kKT;
        int extra = 0;
        // two workgroups on each of the 256 CUs: when the 32-key tiles overflow that by a few
        // tiles per row, fit the row into kLogitsGridSlots / rows tiles, the first of them
        // holding 33 keys (at most one more key per tile)
        const int fit = kLogitsGridSlots / rows_z;
        if (tiles * rows_z > kLogitsGridSlots && fit >= 1 && fit < tiles && max_nkb <= fit * (kKT + 1)) {
            tiles = fit;
            extra = max_nkb - fit * kKT;
        }
        dim3 grid(tiles, s.B * s.Hkv, (s.G * s.Qb + 63) / 64);
        hipLaunchKernelGGL(block_logits_kernel<kKT>, grid, dim3(256), 0, stream, s, qhat, khat, scale, pb, scores,
                           extra);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    SelectParams p;
    p.s = s;
    p.scores = scores;
    p.scores_in = scores_in;
    p.dtype = dtype;
    p.ssb = ssb;
    p.ssh = ssh;
    p.ssq = ssq;
    p.rule = rule;
    p.pb = pb;
    p.rowmask = rowmask;
    const size_t lds = score_select_lds_bytes(s, compute);
    dim3 grid(s.B * s.Hq * s.Qb);
    // rows of up to 16 * 256 blocks (262144 tokens) in registers, longer ones through LDS
    auto launch = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(kSelThreads), lds, stream, p); };
    if (s.cap <= 4 * kSelThreads)
        compute ? launch(row_select_reg_kernel<true, 4>) : launch(row_select_reg_kernel<false, 4>);
    else if (s.cap <= 8 * kSelThreads)
        compute ? launch(row_select_reg_kernel<true, 8>) : launch(row_select_reg_kernel<false, 8>);
    else if (s.cap <= 12 * kSelThreads)
        compute ? launch(row_select_reg_kernel<true, 12>) : launch(row_select_reg_kernel<false, 12>);
    else if (s.cap <= 16 * kSelThreads)
        compute ? launch(row_select_reg_kernel<true, 16>) : launch(row_select_reg_kernel<false, 16>);
    else
        compute ? launch(row_select_kernel<true>) : launch(row_select_kernel<false>);
    return hipGetLastError();
}

hipError_t launch_table_csr(const int32_t* table, int64_t table_stride, const int32_t* counts, int rows, int cap,
                            int32_t* indptr, int32_t* indices, int32_t* last_page_len, hipStream_t stream) {
    CsrParams p;
    p.table = table;
    p.table_stride = table_stride;
    p.counts = counts;
    p.rows = rows;
    p.cap = cap;
    p.indptr = indptr;
    p.indices = indices;
    p.last_page_len = last_page_len;
    hipLaunchKernelGGL(table_csr_kernel, dim3(1), dim3(kCsrThreads), 0, stream, p);
    return hipGetLastError();
}

size_t union_lds_bytes(const Shape& s) { return sizeof(uint32_t) * (size_t)(s.G + 1) * s.words; }

hipError_t launch_union_compact(const Shape& s, const uint32_t* rowmask, int last_n_block,
                                const uint8_t* keep_kv_in, const PastBlocks& pb, uint8_t* keep_block,
                                uint8_t* keep_kv, int32_t* table, int64_t table_stride,
                                int32_t* counts, bool dense, hipStream_t stream) {
    UnionParams p;
    p.s = s;
    p.rowmask = rowmask;
    p.keep_kv_in = keep_kv_in;
    p.mode = dense ? 2 : (keep_kv_in ? 1 : 0);
    int tail = 0;
    if (s.Qb > 1) {
        tail = last_n_block < 0 ? 0 : last_n_block;
        if (tail > s.Qb - 1) tail = s.Qb - 1;
    }
    p.pooled = s.Qb - tail;
    p.pb = pb;
    p.keep_block = keep_block;
    p.keep_kv = keep_kv;
    p.table = table;
    p.table_stride = table_stride;
    p.counts = counts;
    const size_t lds = union_lds_bytes(s);
    hipLaunchKernelGGL(union_compact_kernel, dim3(s.B * s.Hkv), dim3(256), lds, stream, p);
    return hipGetLastError();
}

}  // namespace ca
