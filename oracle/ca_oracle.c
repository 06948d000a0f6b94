/*
 * CPU oracle for the compactattn chunked-prefill path -- TEST INFRASTRUCTURE ONLY
 * (see ca_oracle.h).  Built with -ffp-contract=off: every fused multiply-add below is
 * an explicit fmaf(), every other operation rounds on its own, and sums run in the
 * documented order.  That order is the specification the HIP kernels reproduce.
 *
 * Reference algorithm, per function (paths relative to the reference repository):
 *   orc_block_mean     compact_attn/flashprefill_vendor/flashprefill_native_forward.py:44-95
 *                      (compute_mean_vector: mean of K over each block) and
 *                      compact_attn/prefill_sparse/attn_gate.py:113-130 (avg pooling).
 *   orc_gate_project   compact_attn/prefill_sparse/attn_gate.py:20-34 (MultiHeadLinear,
 *                      einsum 'bshi,hio->bsho'), :132-171 (block RoPE) and
 *                      compact_attn/modules/common.py:29-81 (rotate_half form).
 *   orc_block_scores   compact_attn/prefill_sparse/attn_gate.py:173-204
 *                      (q.k^T * scale, causal block mask, softmax over key blocks) and
 *                      compact_attn/prefill_sparse/llama/modeling_llama_seerattn.py:968-1024
 *                      (block causal mask kb <= floor(q_block_end / 64)); FlashPrefill's
 *                      normalisation over key blocks flashprefill_native_forward.py:365-374.
 *   orc_select_rows    compact_attn/modules/flashprefill_prefill.py:596-666 (alpha over the
 *                      zeroed row :633-645, sink, window, min_budget top-k over all Kb columns
 *                      :637-643, causal :647; and a past-only top-k form), and the Seer rule
 *                      compact_attn/modules/attention_forward_chunked_dense.py:352-403
 *                      (max over valid query blocks > threshold, strict).
 *   orc_union_compact  attention_forward_chunked_dense.py:641-683 (GQA union, current chunk
 *                      open), flashprefill_prefill.py:307-376 (fused union, last_n_block),
 *                      compact_attn/kernels/varlen/flashinfer_zero_copy_prefill.py:482-510
 *                      (ascending selected ids per row).
 *   orc_attention      compact_attn/kernels/varlen/indexed_dense_prefill_direct_triton.py:91-241
 *                      (softmax(q.k*scale).v over the selected blocks, bottom-right causal).
 */
#include "ca_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

int orc_version(void) { return 1; }

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

float orc_bf16_to_f32(uint16_t v) { return bits_f32(((uint32_t)v) << 16); }

uint16_t orc_f32_to_bf16(float v) {
    uint32_t u = f32_bits(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u); /* round to nearest even */
    return (uint16_t)(u >> 16);
}

/* exp(x) by Cody-Waite argument reduction (n = rint(x*log2 e), r = x - n*ln2 split in a
 * high part with trailing zero bits and a low part) and the degree-7 Taylor polynomial of
 * e^r on |r| <= ln2/2 (truncation error < 6e-9 relative), scaled by 2^n built from the
 * exponent bits.  Results below e^-80 are flushed to zero so no subnormal is produced. */
float orc_exp(float x) {
    if (x != x) return x;
    if (x < -80.0f) return 0.0f;
    if (x > 88.0f) return INFINITY;
    const float n = rintf(x * 0x1.715476p+0f);
    float r = fmaf(n, -0x1.62e400p-1f, x);
    r = fmaf(n, -0x1.7f7d1cp-20f, r);
    float p = 1.98412698e-4f;
    p = fmaf(p, r, 1.38888889e-3f);
    p = fmaf(p, r, 8.33333333e-3f);
    p = fmaf(p, r, 4.16666667e-2f);
    p = fmaf(p, r, 1.66666667e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ni = (int)n;
    return p * bits_f32((uint32_t)(ni + 127) << 23);
}

/* Tokens of block n of a sequence of L tokens: 64, or L % 64 for a partial last block. */
static int block_tokens(int L, int n) {
    const int left = L - n * ORC_BLOCK;
    return left < ORC_BLOCK ? left : ORC_BLOCK;
}

/* Block means follow compute_mean_vector (compact_attn/flashprefill_vendor/
 * flashprefill_native_forward.py:44-95): the sum over the block's valid tokens divided by
 * their count (64 except in a partial last block), summed here in token order. */
void orc_block_mean(const uint16_t* x, int B, int L, int H, float* out) {
    const int nb = (L + ORC_BLOCK - 1) / ORC_BLOCK;
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
            for (int n = 0; n < nb; ++n) {
                const int nv = block_tokens(L, n);
                for (int d = 0; d < ORC_D; ++d) {
                    float s = 0.0f;
                    for (int t = 0; t < nv; ++t) {
                        const int64_t tok = (int64_t)n * ORC_BLOCK + t;
                        s = s + orc_bf16_to_f32(x[(((int64_t)b * L + tok) * H + h) * ORC_D + d]);
                    }
                    out[(((int64_t)b * H + h) * nb + n) * ORC_D + d] = s / (float)nv;
                }
            }
}

/* AttnGate pools (attn_gate.py:113-130,233-237; ceil_mode pools cover a partial last block's
 * valid tokens only). */
void orc_block_pool(const uint16_t* x, int B, int L, int H, int pools, float* out) {
    const int nb = (L + ORC_BLOCK - 1) / ORC_BLOCK;
    int C = 0;
    for (int bit = 1; bit <= ORC_POOL_AVG; bit <<= 1) C += (pools & bit) ? 1 : 0;
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
            for (int n = 0; n < nb; ++n) {
                const int nv = block_tokens(L, n);
                float* o = out + (((int64_t)b * H + h) * nb + n) * (int64_t)C * ORC_D;
                for (int d = 0; d < ORC_D; ++d) {
                    const uint16_t* xs = x + ((((int64_t)b * L + (int64_t)n * ORC_BLOCK) * H) + h) * ORC_D + d;
                    const int64_t st = (int64_t)H * ORC_D;
                    float mx = orc_bf16_to_f32(xs[0]), mn = mx, s = 0.0f;
                    for (int t = 0; t < nv; ++t) {
                        const float v = orc_bf16_to_f32(xs[t * st]);
                        mx = v > mx ? v : mx;
                        mn = v < mn ? v : mn;
                        s = s + v;
                    }
                    int c = 0;
                    if (pools & ORC_POOL_MAX) o[(c++) * ORC_D + d] = mx;
                    if (pools & ORC_POOL_MIN) o[(c++) * ORC_D + d] = mn;
                    if (pools & ORC_POOL_AVG) o[(c++) * ORC_D + d] = s / (float)nv;
                }
            }
}

/* 128-token summaries from pairs of 64-token ones: (c0*m0 + c1*m1) / (c0 + c1) in fp32 with the
 * blocks' token counts (64, last_tokens for the last block); an unpaired last block is copied.
 * The order (two products, their sum, one division) is the one the product's pair kernel
 * uses. */
void orc_pair_block_means(const float* src, int rows, int n_blocks, int last_tokens, float* dst) {
    const int np = (n_blocks + 1) / 2;
    for (int r = 0; r < rows; ++r)
        for (int j = 0; j < np; ++j) {
            const int b0 = 2 * j;
            const float* m0 = src + ((int64_t)r * n_blocks + b0) * ORC_D;
            float* o = dst + ((int64_t)r * np + j) * ORC_D;
            if (b0 + 1 >= n_blocks) {
                for (int d = 0; d < ORC_D; ++d) o[d] = m0[d];
                continue;
            }
            const float* m1 = m0 + ORC_D;
            const float c0 = b0 == n_blocks - 1 ? (float)last_tokens : 64.0f;
            const float c1 = b0 + 1 == n_blocks - 1 ? (float)last_tokens : 64.0f;
            const float n = c0 + c1;
            for (int d = 0; d < ORC_D; ++d) {
                const float a = c0 * m0[d];
                const float b = c1 * m1[d];
                const float t = a + b;
                o[d] = t / n;
            }
        }
}

void orc_gate_project(const float* x, int B, int H, int N, const float* W,
                      const float* cos_t, const float* sin_t, int64_t rope_rows,
                      const int32_t* first_block, float* y) {
    orc_gate_project_n(x, B, H, N, ORC_D, W, cos_t, sin_t, rope_rows, first_block, y);
}

void orc_gate_project_n(const float* x, int B, int H, int N, int in, const float* W,
                        const float* cos_t, const float* sin_t, int64_t rope_rows,
                        const int32_t* first_block, float* y) {
    float proj[ORC_D];
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
            for (int n = 0; n < N; ++n) {
                const float* xv = x + (((int64_t)b * H + h) * N + n) * (int64_t)in;
                const float* w = W + (int64_t)h * in * ORC_D;
                for (int o = 0; o < ORC_D; ++o) {
                    float acc = 0.0f;
                    for (int i = 0; i < in; ++i) acc = fmaf(xv[i], w[(int64_t)i * ORC_D + o], acc);
                    proj[o] = acc;
                }
                float* yv = y + (((int64_t)b * H + h) * N + n) * ORC_D;
                if (cos_t == NULL || sin_t == NULL) {
                    memcpy(yv, proj, sizeof(proj));
                    continue;
                }
                const int64_t pos = (int64_t)first_block[b] + n;
                if (pos < 0 || pos >= rope_rows) abort();
                const float* c = cos_t + pos * ORC_D;
                const float* s = sin_t + pos * ORC_D;
                for (int i = 0; i < ORC_D; ++i) {
                    const float rot = (i < ORC_D / 2) ? -proj[i + ORC_D / 2] : proj[i - ORC_D / 2];
                    const float t1 = proj[i] * c[i];
                    const float t2 = rot * s[i];
                    yv[i] = t1 + t2;
                }
            }
}

/* Sum of e[0..n) in the kernels' order: 64 strided partial sums (partial l adds
 * e[l], e[l+64], ... in ascending order), then a halving tree part[l] += part[l+s]
 * for s = 32, 16, ..., 1. */
static float tree64_sum(const float* e, int n) {
    float part[64];
    for (int l = 0; l < 64; ++l) {
        float s = 0.0f;
        for (int i = l; i < n; i += 64) s = s + e[i];
        part[l] = s;
    }
    for (int s = 32; s >= 1; s >>= 1)
        for (int l = 0; l < s; ++l) part[l] = part[l] + part[l + s];
    return part[0];
}

void orc_block_scores(const float* qhat, const float* khat, int B, int Hq, int Hkv, int Qb,
                      int cap, const int32_t* past_blocks, float scale, float* scores) {
    const int G = Hq / Hkv;
    float* logit = (float*)malloc(sizeof(float) * (size_t)cap);
    for (int b = 0; b < B; ++b) {
        const int P = past_blocks[b];
        for (int h = 0; h < Hq; ++h) {
            const int hk = h / G;
            for (int qb = 0; qb < Qb; ++qb) {
                const float* qv = qhat + (((int64_t)b * Hq + h) * Qb + qb) * ORC_D;
                float* srow = scores + (((int64_t)b * Hq + h) * Qb + qb) * cap;
                const int n = P + qb + 1;
                float m = -INFINITY;
                for (int kb = 0; kb < n; ++kb) {
                    const float* kv = khat + (((int64_t)b * Hkv + hk) * cap + kb) * ORC_D;
                    float acc = 0.0f;
                    for (int d = 0; d < ORC_D; ++d) acc = fmaf(qv[d], kv[d], acc);
                    logit[kb] = acc * scale;
                    if (logit[kb] > m) m = logit[kb];
                }
                for (int kb = 0; kb < n; ++kb) logit[kb] = orc_exp(logit[kb] - m);
                const float sum = tree64_sum(logit, n);
                for (int kb = 0; kb < cap; ++kb) srow[kb] = kb < n ? logit[kb] / sum : 0.0f;
            }
        }
    }
    free(logit);
}

static int key_greater(float a, int ia, float b, int ib) {
    /* order by (-score, index): a beats b */
    if (a > b) return 1;
    if (a < b) return 0;
    return ia < ib;
}

/* Value of column kb in the reference's zeroed row (flashprefill_prefill.py:633-634):
 * non-causal (kb > qabs) and non-finite entries read as +0, and -0 is +0. */
static inline float zeroed_value(const float* s, int kb, int n) {
    if (kb >= n || !isfinite(s[kb])) return 0.0f;
    return s[kb] == 0.0f ? 0.0f : s[kb];
}

void orc_select_rows(const float* scores, int B, int Hq, int Qb, int cap,
                     const int32_t* past_blocks, const orc_rule* rule, uint8_t* rowkeep) {
    int* cand = (int*)malloc(sizeof(int) * (size_t)(cap > 0 ? cap : 1));
    float* val = (float*)malloc(sizeof(float) * (size_t)(cap > 0 ? cap : 1));
    const int all_cols = (rule->flags & ORC_RULE_TOPK_ALLCOLS) != 0;
    for (int b = 0; b < B; ++b) {
        const int P = past_blocks[b];
        const int Kb = P + Qb;
        for (int h = 0; h < Hq; ++h)
            for (int qb = 0; qb < Qb; ++qb) {
                const float* s = scores + (((int64_t)b * Hq + h) * Qb + qb) * cap;
                uint8_t* out = rowkeep + (((int64_t)b * Hq + h) * Qb + qb) * cap;
                const int qabs = P + qb;
                const int n = qabs + 1; /* causal columns */
                memset(out, 0, (size_t)cap);
                /* alpha rule: the max over all Kb columns of the zeroed row (:633-645) */
                float rowmax = zeroed_value(s, 0, n);
                for (int kb = 1; kb < Kb; ++kb) {
                    const float v = zeroed_value(s, kb, n);
                    if (v > rowmax) rowmax = v;
                }
                const float alpha_cut = rule->alpha * rowmax;
                for (int kb = 0; kb < n; ++kb) {
                    int keep = 0;
                    const int fin = isfinite(s[kb]);
                    if ((rule->flags & ORC_RULE_ALPHA) && fin && s[kb] >= alpha_cut) keep = 1;
                    if ((rule->flags & ORC_RULE_THRESHOLD) && s[kb] > rule->threshold) keep = 1;
                    if (kb < rule->sink_blocks) keep = 1;
                    if (qabs - kb < rule->window_blocks) keep = 1;
                    if (kb < P && kb >= P - rule->local_blocks) keep = 1;
                    out[kb] = (uint8_t)keep;
                }
                if ((rule->flags & ORC_RULE_TOPK) && rule->topk > 0) {
                    /* Candidates by (-score, index), taken by repeated extraction of the best
                     * remaining one.
                     *  - past-only form: the finite past blocks kb < P;
                     *  - all-columns form (the reference's min_budget, torch.topk over the Kb
                     *    columns of the zeroed row, :637-643): every kb < Kb with its zeroed
                     *    value; picks past the causal edge are dropped by the causal mask (:647). */
                    int nc = 0;
                    if (all_cols) {
                        for (int kb = 0; kb < Kb; ++kb) {
                            val[kb] = zeroed_value(s, kb, n);
                            cand[nc++] = kb;
                        }
                    } else {
                        for (int kb = 0; kb < P && kb < n; ++kb)
                            if (isfinite(s[kb])) {
                                val[kb] = s[kb] == 0.0f ? 0.0f : s[kb];
                                cand[nc++] = kb;
                            }
                    }
                    const int k = rule->topk < nc ? rule->topk : nc;
                    for (int i = 0; i < k; ++i) {
                        int best = i;
                        for (int j = i + 1; j < nc; ++j)
                            if (key_greater(val[cand[j]], cand[j], val[cand[best]], cand[best])) best = j;
                        const int tmp = cand[i];
                        cand[i] = cand[best];
                        cand[best] = tmp;
                        if (cand[i] < n) out[cand[i]] = 1;
                    }
                }
            }
    }
    free(val);
    free(cand);
}

void orc_union_compact(const uint8_t* rowkeep, int B, int Hq, int Hkv, int Qb, int cap,
                       const int32_t* past_blocks, int last_n_block, uint8_t* keep_block,
                       uint8_t* keep_kv, int32_t* table, int32_t* counts) {
    const int G = Hq / Hkv;
    int tail = 0;
    if (Qb > 1) {
        tail = last_n_block < 0 ? 0 : last_n_block;
        if (tail > Qb - 1) tail = Qb - 1;
    }
    const int pooled = Qb - tail;
    for (int b = 0; b < B; ++b) {
        const int P = past_blocks[b];
        const int Kb = P + Qb;
        for (int h = 0; h < Hq; ++h) {
            uint8_t* kbk = keep_block + ((int64_t)b * Hq + h) * cap;
            memset(kbk, 0, (size_t)cap);
            for (int kb = 0; kb < Kb; ++kb) {
                int any = kb >= P;
                for (int qb = 0; qb < pooled && !any; ++qb)
                    any = rowkeep[(((int64_t)b * Hq + h) * Qb + qb) * cap + kb] != 0;
                kbk[kb] = (uint8_t)any;
            }
        }
        for (int hk = 0; hk < Hkv; ++hk) {
            uint8_t* kv = keep_kv + ((int64_t)b * Hkv + hk) * cap;
            int32_t* tab = table + ((int64_t)b * Hkv + hk) * cap;
            memset(kv, 0, (size_t)cap);
            int c = 0;
            for (int kb = 0; kb < Kb; ++kb) {
                int any = 0;
                for (int g = 0; g < G; ++g) any |= keep_block[((int64_t)b * Hq + hk * G + g) * cap + kb];
                kv[kb] = (uint8_t)any;
                if (any) tab[c++] = kb;
            }
            for (int i = c; i < cap; ++i) tab[i] = -1;
            counts[(int64_t)b * Hkv + hk] = c;
        }
    }
}

void orc_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, int B, int Lq, int Hq,
                   int Hkv, int cap, const int32_t* past_blocks, const int32_t* table,
                   const int32_t* counts, float scale, int q_begin, int q_end, int head_begin,
                   int head_end, float* out, float* lse) {
    const int G = Hq / Hkv;
    const int64_t ktok = (int64_t)cap * ORC_BLOCK;
    const int nh = head_end - head_begin;
    const int nq = q_end - q_begin;
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
    for (int bh = 0; bh < B * nh; ++bh)
        for (int t = q_begin; t < q_end; ++t) {
            const int b = bh / nh;
            const int h = head_begin + bh % nh;
            const int hk = h / G;
            const int row = b * Hkv + hk;
            const int P = past_blocks[b];
            const int64_t qpos = (int64_t)P * ORC_BLOCK + t;
            const int cnt = counts[row];
            const int32_t* tab = table + (int64_t)row * cap;
            double qd[ORC_D];
            const uint16_t* qv = q + (((int64_t)b * Lq + t) * Hq + h) * ORC_D;
            for (int d = 0; d < ORC_D; ++d) qd[d] = orc_bf16_to_f32(qv[d]);
            double* sc = (double*)malloc(sizeof(double) * (size_t)cnt * ORC_BLOCK);
            double m = -INFINITY;
            for (int e = 0; e < cnt; ++e) {
                const int kb = tab[e];
                for (int j = 0; j < ORC_BLOCK; ++j) {
                    const int64_t kpos = (int64_t)kb * ORC_BLOCK + j;
                    double s = -INFINITY;
                    if (kpos <= qpos) {
                        const uint16_t* kv = k + ((int64_t)row * ktok + kpos) * ORC_D;
                        double acc = 0.0;
                        for (int d = 0; d < ORC_D; ++d) acc += qd[d] * orc_bf16_to_f32(kv[d]);
                        s = acc * (double)scale;
                        if (s > m) m = s;
                    }
                    sc[(int64_t)e * ORC_BLOCK + j] = s;
                }
            }
            double o[ORC_D];
            for (int d = 0; d < ORC_D; ++d) o[d] = 0.0;
            double l = 0.0;
            for (int e = 0; e < cnt; ++e) {
                const int kb = tab[e];
                for (int j = 0; j < ORC_BLOCK; ++j) {
                    const double s = sc[(int64_t)e * ORC_BLOCK + j];
                    if (s == -INFINITY) continue;
                    const double p = exp(s - m);
                    l += p;
                    const uint16_t* vv = v + ((int64_t)row * ktok + (int64_t)kb * ORC_BLOCK + j) * ORC_D;
                    for (int d = 0; d < ORC_D; ++d) o[d] += p * orc_bf16_to_f32(vv[d]);
                }
            }
            free(sc);
            float* ov = out + (((int64_t)b * Lq + t) * Hq + h) * ORC_D;
            for (int d = 0; d < ORC_D; ++d) ov[d] = (float)(l > 0.0 ? o[d] / l : 0.0);
            if (lse) lse[((int64_t)b * Hq + h) * Lq + t] = (float)(l > 0.0 ? m + log(l) : -INFINITY);
        }
    (void)nq;
}
