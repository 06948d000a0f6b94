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
// Gate projection (per-head 128x128, y[o] = sum_i x[i] W[i][o], sequential fma over i) and
// block RoPE y[i] = x[i] cos[i] + rotate_half(x)[i] sin[i].  64 threads; thread t owns the
// output pair (t, t + 64), which is exactly a rotate_half pair.
__device__ void gate_project_rope(const float* xs, const float* w, const float* rope_cos,
                                  const float* rope_sin, int64_t pos, float* out) {
    const int t = threadIdx.x;
    float a0 = 0.0f, a1 = 0.0f;
    for (int i = 0; i < kD; ++i) {
        const float x = xs[i];
        a0 = __builtin_fmaf(x, w[i * kD + t], a0);
        a1 = __builtin_fmaf(x, w[i * kD + t + 64], a1);
    }
    if (rope_cos == nullptr) {
        out[t] = a0;
        out[t + 64] = a1;
        return;
    }
    const float* c = rope_cos + pos * kD;
    const float* s = rope_sin + pos * kD;
    {
        const float t1 = a0 * c[t];
        const float t2 = (-a1) * s[t];
        out[t] = t1 + t2;
    }
    {
        const float t1 = a1 * c[t + 64];
        const float t2 = a0 * s[t + 64];
        out[t + 64] = t1 + t2;
    }
}

// ---------------------------------------------------------------------------------------
// Cache fill: one 64-token block of one (request, KV head) per workgroup.  Threads 0..63 copy
// K (two head-dim lanes each) and accumulate the block mean; threads 64..127 copy V.
__global__ __launch_bounds__(128) void cache_fill_kernel(Shape s, SeqAddr kn, SeqAddr vn,
                                                         KvAddr kc, KvAddr vc, PastBlocks pb,
                                                         float* kmean, const float* wk,
                                                         const float* rope_cos,
                                                         const float* rope_sin, float* kgate) {
    const int j = blockIdx.x;
    const int row = blockIdx.y;
    const int b = row / s.Hkv;
    const int hk = row - b * s.Hkv;
    const int kb = pb.p[b] + j;
    const bool is_v = threadIdx.x >= 64;
    const int lane = threadIdx.x & 63;
    const SeqAddr& src = is_v ? vn : kn;
    const KvAddr& dst = is_v ? vc : kc;
    const int64_t phys = dst.page_table ? dst.page_table[(int64_t)row * dst.pts + kb] : kb;
    const uint16_t* sp = src.data + b * src.sb + (int64_t)j * kBlock * src.st + hk * src.sh + 2 * lane;
    uint16_t* dp = dst.data + b * dst.sb + hk * dst.sh + phys * dst.sblk + 2 * lane;
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll 8
    for (int t = 0; t < kBlock; ++t) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(sp + t * src.st);
        *reinterpret_cast<uint32_t*>(dp + t * dst.stok) = v;
        s0 = s0 + bf16_to_f32(static_cast<uint16_t>(v & 0xffffu));
        s1 = s1 + bf16_to_f32(static_cast<uint16_t>(v >> 16));
    }
    __shared__ float xs[kD];
    const int64_t srow = ((int64_t)row * s.cap + kb) * kD;
    if (!is_v) {
        const float m0 = s0 * 0.015625f;
        const float m1 = s1 * 0.015625f;
        if (kmean) {
            kmean[srow + 2 * lane] = m0;
            kmean[srow + 2 * lane + 1] = m1;
        }
        xs[2 * lane] = m0;
        xs[2 * lane + 1] = m1;
    }
    if (wk == nullptr) return;
    __syncthreads();
    if (!is_v) gate_project_rope(xs, wk + (int64_t)hk * kD * kD, rope_cos, rope_sin, kb, kgate + srow);
}

// ---------------------------------------------------------------------------------------
// Query-block means (optionally gate-projected and rotated): one (block, request, head) per
// workgroup of 64 threads, two head-dim lanes per thread.
__global__ __launch_bounds__(64) void pool_query_kernel(Shape s, SeqAddr q, PastBlocks pb,
                                                        const float* wq, const float* rope_cos,
                                                        const float* rope_sin, float* qhat) {
    const int qb = blockIdx.x;
    const int bh = blockIdx.y;
    const int b = bh / s.Hq;
    const int h = bh - b * s.Hq;
    const int lane = threadIdx.x;
    const uint16_t* sp = q.data + b * q.sb + (int64_t)qb * kBlock * q.st + h * q.sh + 2 * lane;
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll 8
    for (int t = 0; t < kBlock; ++t) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(sp + t * q.st);
        s0 = s0 + bf16_to_f32(static_cast<uint16_t>(v & 0xffffu));
        s1 = s1 + bf16_to_f32(static_cast<uint16_t>(v >> 16));
    }
    float* out = qhat + ((int64_t)bh * s.Qb + qb) * kD;
    const float m0 = s0 * 0.015625f;
    const float m1 = s1 * 0.015625f;
    if (wq == nullptr) {
        out[2 * lane] = m0;
        out[2 * lane + 1] = m1;
        return;
    }
    __shared__ float xs[kD];
    xs[2 * lane] = m0;
    xs[2 * lane + 1] = m1;
    __syncthreads();
    gate_project_rope(xs, wq + (int64_t)h * kD * kD, rope_cos, rope_sin, (int64_t)pb.p[b] + qb, out);
}

// ---------------------------------------------------------------------------------------
// Scoring + selection.  One workgroup (256 threads) per (request, KV head, query block)
// handles the G rows of the group's Q heads.
constexpr int kPadRow = kD + 4;  // LDS row pitch (floats) for summary tiles

__device__ __forceinline__ int score_tile_rows(int G) {
    const int r = 256 / G;
    return r < 64 ? r : 64;
}

struct SelectParams {
    Shape s;
    const float* qhat;
    const float* khat;
    float scale;
    const void* scores_in;
    int dtype;
    int64_t ssb, ssh, ssq;
    ca_select_rule rule;
    PastBlocks pb;
    uint32_t* rowmask;
    float* scores_out;
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

template <bool kCompute>
__global__ __launch_bounds__(256) void score_select_kernel(SelectParams p) {
    extern __shared__ float lds[];
    __shared__ float red[256];
    __shared__ int ired[8];
    __shared__ int hist[256];
    __shared__ int sel_digit, sel_above;

    const Shape& s = p.s;
    const int qb = blockIdx.x;
    const int row = blockIdx.y;
    const int b = row / s.Hkv;
    const int hk = row - b * s.Hkv;
    const int G = s.G;
    const int t = threadIdx.x;
    const int P = p.pb.p[b];
    const int qabs = P + qb;
    const int n = qabs + 1;  // causal columns
    const int cap = s.cap;
    float* sc = lds;  // [G][cap]

    if (kCompute) {
        float* qv = lds + (size_t)G * cap;  // [G][kPadRow]
        float* kt = qv + (size_t)G * kPadRow;  // [TK][kPadRow]
        const int TK = score_tile_rows(G);
        for (int i = t; i < G * kD; i += 256) {
            const int g = i / kD, d = i - g * kD;
            qv[g * kPadRow + d] =
                p.qhat[(((int64_t)b * s.Hq + hk * G + g) * s.Qb + qb) * kD + d];
        }
        const float* kbase = p.khat + (int64_t)row * cap * kD;
        for (int kb0 = 0; kb0 < n; kb0 += TK) {
            const int rows_here = min(TK, n - kb0);
            __syncthreads();
            for (int f = t; f < rows_here * (kD / 4); f += 256) {
                const int r = f >> 5, c4 = f & 31;
                const float4 v = *reinterpret_cast<const float4*>(kbase + (int64_t)(kb0 + r) * kD + c4 * 4);
                *reinterpret_cast<float4*>(kt + r * kPadRow + c4 * 4) = v;
            }
            __syncthreads();
            if (t < TK * G) {
                const int kl = t / G, g = t - kl * G;
                if (kl < rows_here) {
                    const float* a = qv + g * kPadRow;
                    const float* k = kt + kl * kPadRow;
                    float acc = 0.0f;
#pragma unroll 16
                    for (int d = 0; d < kD; ++d) acc = __builtin_fmaf(a[d], k[d], acc);
                    sc[g * cap + kb0 + kl] = acc * p.scale;
                }
            }
        }
        __syncthreads();
        // softmax over the causal columns of each row
        for (int g = 0; g < G; ++g) {
            float* r = sc + g * cap;
            float m = -__builtin_inff();
            for (int kb = t; kb < n; kb += 256) m = fmaxf(m, r[kb]);
            m = block_max256(m, red);
            float part = 0.0f;
            for (int kb = t; kb < n; kb += 256) {
                const float e = exp_fixed(r[kb] - m);
                r[kb] = e;
                part = part + e;
            }
            const float sum = tree256_sum(part, red);
            for (int kb = t; kb < n; kb += 256) r[kb] = r[kb] / sum;
            if (p.scores_out) {
                float* o = p.scores_out + (((int64_t)b * s.Hq + hk * G + g) * s.Qb + qb) * cap;
                for (int kb = t; kb < cap; kb += 256) o[kb] = kb < n ? r[kb] : 0.0f;
            }
        }
        __syncthreads();
    } else {
        for (int g = 0; g < G; ++g) {
            const int h = hk * G + g;
            const int64_t off = b * p.ssb + h * p.ssh + qb * p.ssq;
            for (int kb = t; kb < n; kb += 256) {
                float v;
                if (p.dtype == 0)
                    v = static_cast<const float*>(p.scores_in)[off + kb];
                else
                    v = bf16_to_f32(static_cast<const uint16_t*>(p.scores_in)[off + kb]);
                sc[g * cap + kb] = v;
            }
        }
        __syncthreads();
    }

    // ---- selection, one row at a time ----
    const ca_select_rule& rule = p.rule;
    const bool use_topk = (rule.flags & CA_RULE_TOPK) && rule.topk > 0 && P > 0;
    const int chunks = (s.words * 32 + 255) / 256;
    const int wave = t >> 6, lane = t & 63;
    for (int g = 0; g < G; ++g) {
        const float* r = sc + g * cap;
        float mx = 0.0f;
        for (int kb = t; kb < n; kb += 256) {
            const float v = r[kb];
            if (is_finite_f(v)) mx = fmaxf(mx, v);
        }
        const float rowmax = block_max256(mx, red);
        const float alpha_cut = rule.alpha * rowmax;

        // top-k threshold key T and the number of ties at T to take (lowest ids first)
        bool take_all = false;
        uint32_t T = 0;
        int krem = 0;
        if (use_topk) {
            int nc = 0;
            for (int kb = t; kb < P; kb += 256) nc += is_finite_f(r[kb]) ? 1 : 0;
            nc = block_sum256_int(nc, ired);
            if (rule.topk >= nc) {
                take_all = true;
            } else {
                uint32_t prefix = 0, pmask = 0;
                krem = rule.topk;
                for (int shift = 24; shift >= 0; shift -= 8) {
                    hist[t] = 0;
                    __syncthreads();
                    for (int kb = t; kb < P; kb += 256) {
                        const float v = r[kb];
                        if (!is_finite_f(v)) continue;
                        const uint32_t key = order_key(v);
                        if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
                    }
                    __syncthreads();
                    // suffix counts from the top digit down: thread t looks at digit 255 - t
                    const int hcount = hist[255 - t];
                    int tot;
                    const int excl = block_exclusive_scan256(hcount, ired, &tot);
                    if (hcount > 0 && excl < krem && krem <= excl + hcount) {
                        sel_digit = 255 - t;
                        sel_above = excl;
                    }
                    __syncthreads();
                    prefix |= static_cast<uint32_t>(sel_digit) << shift;
                    pmask |= 255u << shift;
                    krem -= sel_above;
                    __syncthreads();
                }
                T = prefix;
            }
        }

        const int h = hk * G + g;
        uint32_t* out = p.rowmask + (((int64_t)b * s.Hq + h) * s.Qb + qb) * s.words;
        int eq_base = 0;
        for (int c = 0; c < chunks; ++c) {
            const int kb = c * 256 + t;
            bool keep = false;
            bool eq = false;
            if (kb < n) {
                const float v = r[kb];
                const bool fin = is_finite_f(v);
                if ((rule.flags & CA_RULE_ALPHA) && fin && v >= alpha_cut) keep = true;
                if ((rule.flags & CA_RULE_THRESHOLD) && v > rule.threshold) keep = true;
                if (kb < rule.sink_blocks) keep = true;
                if (qabs - kb < rule.window_blocks) keep = true;
                if (kb < P && kb >= P - rule.local_blocks) keep = true;
                if (use_topk && kb < P && fin) {
                    if (take_all) {
                        keep = true;
                    } else {
                        const uint32_t key = order_key(v);
                        if (key > T) keep = true;
                        eq = key == T;
                    }
                }
            }
            if (use_topk && !take_all) {
                int tot;
                const int rank = block_exclusive_scan256(eq ? 1 : 0, ired, &tot);
                if (eq && eq_base + rank < krem) keep = true;
                eq_base += tot;
            }
            const uint64_t bal = __ballot(keep);
            const int w0 = (c * 256 + wave * 64) >> 5;
            if (lane == 0 && w0 < s.words) out[w0] = static_cast<uint32_t>(bal);
            if (lane == 1 && w0 + 1 < s.words) out[w0 + 1] = static_cast<uint32_t>(bal >> 32);
        }
        __syncthreads();
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
    extern __shared__ uint32_t kvw[];
    __shared__ int ired[8];
    const Shape& s = p.s;
    const int row = blockIdx.x;
    const int b = row / s.Hkv;
    const int hk = row - b * s.Hkv;
    const int t = threadIdx.x;
    const int P = p.pb.p[b];
    const int nkb = P + s.Qb;
    const int G = s.G;
    for (int w = t; w < s.words; w += 256) {
        const uint32_t valid = range_bits(w, 0, nkb);
        const uint32_t cur = range_bits(w, P, nkb);
        uint32_t acc = 0;
        if (p.mode == 0) {
            for (int g = 0; g < G; ++g) {
                const int h = hk * G + g;
                uint32_t hw = cur;
                const uint32_t* rm = p.rowmask + ((int64_t)b * s.Hq + h) * s.Qb * s.words + w;
                for (int qb = 0; qb < p.pooled; ++qb) hw |= rm[(int64_t)qb * s.words];
                hw &= valid;
                if (p.keep_block) {
                    uint8_t* kbk = p.keep_block + ((int64_t)b * s.Hq + h) * s.cap + 32 * w;
                    for (int i = 0; i < 32 && 32 * w + i < s.cap; ++i) kbk[i] = (hw >> i) & 1u;
                }
                acc |= hw;
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
    const int wpt = (s.words + 255) / 256;
    const int w0 = t * wpt;
    const int w1 = min(w0 + wpt, s.words);
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

}  // namespace

hipError_t launch_cache_fill(const Shape& s, const SeqAddr& k_new, const SeqAddr& v_new,
                             const KvAddr& k_cache, const KvAddr& v_cache, const PastBlocks& pb,
                             float* kmean, const float* wk, const float* rope_cos,
                             const float* rope_sin, float* kgate, hipStream_t stream) {
    dim3 grid(s.Qb, s.B * s.Hkv);
    hipLaunchKernelGGL(cache_fill_kernel, grid, dim3(128), 0, stream, s, k_new, v_new, k_cache,
                       v_cache, pb, kmean, wk, rope_cos, rope_sin, kgate);
    return hipGetLastError();
}

hipError_t launch_pool_query(const Shape& s, const SeqAddr& q, const PastBlocks& pb, const float* wq,
                             const float* rope_cos, const float* rope_sin, float* qhat,
                             hipStream_t stream) {
    dim3 grid(s.Qb, s.B * s.Hq);
    hipLaunchKernelGGL(pool_query_kernel, grid, dim3(64), 0, stream, s, q, pb, wq, rope_cos,
                       rope_sin, qhat);
    return hipGetLastError();
}

size_t score_select_lds_bytes(const Shape& s, bool compute) {
    size_t bytes = sizeof(float) * (size_t)s.G * s.cap;
    if (compute) {
        const int tk = (256 / s.G) < 64 ? 256 / s.G : 64;
        bytes += sizeof(float) * (size_t)(s.G + tk) * kPadRow;
    }
    return bytes;
}

hipError_t launch_score_select(const Shape& s, const float* qhat, const float* khat, float scale,
                               const void* scores_in, int dtype, int64_t ssb, int64_t ssh,
                               int64_t ssq, const ca_select_rule& rule, const PastBlocks& pb,
                               uint32_t* rowmask, float* scores_out, hipStream_t stream) {
    SelectParams p;
    p.s = s;
    p.qhat = qhat;
    p.khat = khat;
    p.scale = scale;
    p.scores_in = scores_in;
    p.dtype = dtype;
    p.ssb = ssb;
    p.ssh = ssh;
    p.ssq = ssq;
    p.rule = rule;
    p.pb = pb;
    p.rowmask = rowmask;
    p.scores_out = scores_out;
    const bool compute = scores_in == nullptr;
    const size_t lds = score_select_lds_bytes(s, compute);
    dim3 grid(s.Qb, s.B * s.Hkv);
    if (compute) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(score_select_kernel<true>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(score_select_kernel<true>, grid, dim3(256), lds, stream, p);
    } else {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(score_select_kernel<false>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(score_select_kernel<false>, grid, dim3(256), lds, stream, p);
    }
    return hipGetLastError();
}

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
    const size_t lds = sizeof(uint32_t) * (size_t)s.words;
    hipLaunchKernelGGL(union_compact_kernel, dim3(s.B * s.Hkv), dim3(256), lds, stream, p);
    return hipGetLastError();
}

}  // namespace ca
