// C-ABI entry points of libcompactattn_hip.so: host-side argument validation, then the
// kernel launches on the caller's stream.  No device allocation, no host synchronisation.
// Declarations and reference citations are in include/compactattn.h.

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/compactattn.h"
#include "ca_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok() {
    g_last_error.clear();
    return CA_OK;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(CA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int64_t kMaxStrideTok = int64_t{1} << 24;  // 64 rows x 2 bytes x stride_tok < 2^31

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

// Validates dims + past blocks and fills the internal shape.
int check_dims(const ca_dims* d, const int32_t* past_host, ca::Shape* s, ca::PastBlocks* pb,
               int* max_nkb) {
    if (d == nullptr) return fail(CA_ERR_INVALID, "dims is NULL");
    if (past_host == nullptr) return fail(CA_ERR_INVALID, "past_blocks_host is NULL");
    if (d->batch < 1 || d->batch > CA_MAX_BATCH)
        return fail(d->batch < 1 ? CA_ERR_INVALID : CA_ERR_LIMIT, "batch=%d outside [1, %d]",
                    d->batch, CA_MAX_BATCH);
    if (d->q_len <= 0) return fail(CA_ERR_INVALID, "q_len=%d must be positive", d->q_len);
    if (d->num_q_heads <= 0 || d->num_kv_heads <= 0 || d->num_q_heads % d->num_kv_heads != 0)
        return fail(CA_ERR_INVALID, "num_q_heads=%d must be a positive multiple of num_kv_heads=%d",
                    d->num_q_heads, d->num_kv_heads);
    const int G = d->num_q_heads / d->num_kv_heads;
    if (G > 16) return fail(CA_ERR_LIMIT, "GQA group size %d > 16", G);
    // the chunk's blocks: the last one holds q_len % 64 tokens when q_len is not a multiple of 64
    const int Qb = (d->q_len + CA_BLOCK - 1) / CA_BLOCK;
    int mx = 0;
    for (int b = 0; b < d->batch; ++b) {
        if (past_host[b] < 0) return fail(CA_ERR_INVALID, "past_blocks[%d]=%d < 0", b, past_host[b]);
        if ((int64_t)past_host[b] + Qb > d->kv_cap)
            return fail(CA_ERR_INVALID, "past_blocks[%d]=%d + ceil(q_len/64)=%d exceeds kv_cap=%d", b,
                        past_host[b], Qb, d->kv_cap);
        pb->p[b] = past_host[b];
        if (past_host[b] + Qb > mx) mx = past_host[b] + Qb;
    }
    for (int b = d->batch; b < CA_MAX_BATCH; ++b) pb->p[b] = 0;
    if ((int64_t)d->kv_cap * CA_BLOCK > (int64_t)1 << 30)
        return fail(CA_ERR_LIMIT, "kv_cap=%d blocks too large", d->kv_cap);
    s->B = d->batch;
    s->Lq = d->q_len;
    s->Hq = d->num_q_heads;
    s->Hkv = d->num_kv_heads;
    s->G = G;
    s->Qb = Qb;
    s->cap = d->kv_cap;
    s->words = (d->kv_cap + 31) / 32;
    *max_nkb = mx;
    return CA_OK;
}

// Validates dims + per-request KV lengths of a decode call (q_len query rows per request
// sit at the last q_len positions of its kv_len tokens) and fills the internal shape.
int check_decode_dims(const ca_dims* d, const int32_t* kv_len, ca::Shape* s, ca::PastBlocks* pb,
                      int* max_nkb) {
    if (d == nullptr) return fail(CA_ERR_INVALID, "dims is NULL");
    if (kv_len == nullptr) return fail(CA_ERR_INVALID, "kv_len_host is NULL");
    if (d->batch < 1 || d->batch > CA_MAX_BATCH)
        return fail(d->batch < 1 ? CA_ERR_INVALID : CA_ERR_LIMIT, "batch=%d outside [1, %d]",
                    d->batch, CA_MAX_BATCH);
    if (d->q_len < 1 || d->q_len > CA_BLOCK)
        return fail(CA_ERR_INVALID, "decode q_len=%d outside [1, %d]", d->q_len, CA_BLOCK);
    if (d->num_q_heads <= 0 || d->num_kv_heads <= 0 || d->num_q_heads % d->num_kv_heads != 0)
        return fail(CA_ERR_INVALID, "num_q_heads=%d must be a positive multiple of num_kv_heads=%d",
                    d->num_q_heads, d->num_kv_heads);
    const int G = d->num_q_heads / d->num_kv_heads;
    if (G > 16) return fail(CA_ERR_LIMIT, "GQA group size %d > 16", G);
    if (d->kv_cap < 1 || (int64_t)d->kv_cap * CA_BLOCK > (int64_t)1 << 30)
        return fail(d->kv_cap < 1 ? CA_ERR_INVALID : CA_ERR_LIMIT, "kv_cap=%d blocks outside [1, 2^24]", d->kv_cap);
    int mx = 0;
    for (int b = 0; b < d->batch; ++b) {
        if (kv_len[b] < d->q_len || (int64_t)kv_len[b] > (int64_t)d->kv_cap * CA_BLOCK)
            return fail(CA_ERR_INVALID, "kv_len[%d]=%d outside [q_len=%d, 64 * kv_cap=%lld]", b, kv_len[b],
                        d->q_len, (long long)d->kv_cap * CA_BLOCK);
        mx = max(mx, (kv_len[b] + CA_BLOCK - 1) / CA_BLOCK);
        pb->p[b] = 0;
    }
    for (int b = d->batch; b < CA_MAX_BATCH; ++b) pb->p[b] = 0;
    s->B = d->batch;
    s->Lq = d->q_len;
    s->Hq = d->num_q_heads;
    s->Hkv = d->num_kv_heads;
    s->G = G;
    s->Qb = 0;
    s->cap = d->kv_cap;
    s->words = (d->kv_cap + 31) / 32;
    *max_nkb = mx;
    return CA_OK;
}

int check_seq(const ca_seq_layout* l, const char* name, ca::SeqAddr* out) {
    if (l == nullptr || l->data == nullptr) return fail(CA_ERR_INVALID, "%s is NULL", name);
    if (!aligned16(l->data)) return fail(CA_ERR_INVALID, "%s data must be 16-byte aligned", name);
    if (l->stride_b % 8 || l->stride_t % 8 || l->stride_h % 8 || l->stride_t <= 0 || l->stride_h <= 0 ||
        l->stride_b < 0)
        return fail(CA_ERR_INVALID, "%s strides (b=%lld, t=%lld, h=%lld) must be multiples of 8 and t,h > 0",
                    name, (long long)l->stride_b, (long long)l->stride_t, (long long)l->stride_h);
    out->data = static_cast<uint16_t*>(l->data);
    out->sb = l->stride_b;
    out->st = l->stride_t;
    out->sh = l->stride_h;
    return CA_OK;
}

int check_kv(const ca_kv_layout* l, const char* name, int max_nkb, ca::KvAddr* out) {
    if (l == nullptr || l->data == nullptr) return fail(CA_ERR_INVALID, "%s is NULL", name);
    if (!aligned16(l->data)) return fail(CA_ERR_INVALID, "%s data must be 16-byte aligned", name);
    if (l->stride_b % 8 || l->stride_h % 8 || l->stride_blk % 8 || l->stride_tok % 8 || l->stride_tok <= 0 ||
        l->stride_b < 0 || l->stride_h < 0 || l->stride_blk < 0)
        return fail(CA_ERR_INVALID, "%s strides must be non-negative multiples of 8 (stride_tok > 0)", name);
    // the kernels address a block's rows with 32-bit byte offsets (up to 64 * 2 * stride_tok)
    if (l->stride_tok >= kMaxStrideTok)
        return fail(CA_ERR_LIMIT, "%s stride_tok=%lld: a 64-token block must span < 2^31 bytes (stride_tok < %lld)",
                    name, (long long)l->stride_tok, (long long)kMaxStrideTok);
    if (l->page_table != nullptr) {
        if (!aligned4(l->page_table)) return fail(CA_ERR_INVALID, "%s page_table misaligned", name);
        if (l->page_table_stride < max_nkb)
            return fail(CA_ERR_INVALID, "%s page_table_stride=%lld < blocks per row %d", name,
                        (long long)l->page_table_stride, max_nkb);
        if (l->num_pages < 1 || l->num_pages > INT32_MAX)
            return fail(CA_ERR_INVALID, "%s num_pages=%lld must be in [1, 2^31) with a page table", name,
                        (long long)l->num_pages);
    }
    out->data = static_cast<uint16_t*>(l->data);
    out->sb = l->stride_b;
    out->sh = l->stride_h;
    out->sblk = l->stride_blk;
    out->stok = l->stride_tok;
    out->page_table = l->page_table;
    out->pts = l->page_table_stride;
    out->max_page = l->page_table != nullptr ? static_cast<int32_t>(l->num_pages - 1) : 0;
    return CA_OK;
}

int check_rope(const float* c, const float* s, int64_t rows, int max_nkb) {
    if ((c == nullptr) != (s == nullptr)) return fail(CA_ERR_INVALID, "rope_cos and rope_sin must both be set or both NULL");
    if (c != nullptr && rows < max_nkb)
        return fail(CA_ERR_INVALID, "rope_rows=%lld < highest block id + 1 = %d", (long long)rows, max_nkb);
    if (c != nullptr && (!aligned4(c) || !aligned4(s))) return fail(CA_ERR_INVALID, "rope tables misaligned");
    return CA_OK;
}

int check_pools(int32_t pools) {
    if (pools <= 0 || (pools & ~(CA_POOL_MAX | CA_POOL_MIN | CA_POOL_AVG)))
        return fail(CA_ERR_INVALID, "pools=0x%x must be a non-empty set of CA_POOL_MAX/MIN/AVG", pools);
    return CA_OK;
}

int check_rule(const ca_select_rule* r) {
    if (r == nullptr) return fail(CA_ERR_INVALID, "rule is NULL");
    if (r->flags & ~(CA_RULE_TOPK | CA_RULE_ALPHA | CA_RULE_THRESHOLD | CA_RULE_TOPK_ALLCOLS))
        return fail(CA_ERR_INVALID, "unknown rule flags 0x%x", r->flags);
    if ((r->flags & CA_RULE_TOPK_ALLCOLS) && !(r->flags & CA_RULE_TOPK))
        return fail(CA_ERR_INVALID, "CA_RULE_TOPK_ALLCOLS needs CA_RULE_TOPK");
    if ((r->flags & CA_RULE_TOPK) && r->topk < 0) return fail(CA_ERR_INVALID, "topk=%d < 0", r->topk);
    return CA_OK;
}

constexpr size_t kMaxLds = 160 * 1024 - 4096;  // dynamic LDS budget next to static arrays

// ---- scratch of the allocation-free entry point (ca_attn_fwd_noalloc) ----
// The split partials live in this file-scope device array: every GPU the library runs on
// holds its own copy until the process ends.  In host code the name is only a host-side
// handle; the array's address on a device comes from hipGetSymbolAddress with that device
// current, looked up once per device and kept here.  Every call on a GPU shares its array
// (calls that overlap on one GPU race); the attention kernel writes every partial row the
// merge reads, so nothing needs clearing between calls.
static __device__ __align__(256) uint8_t scratch[CA_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The scratch array's address on the device of `stream` (the current device, which must be
// the stream's device).
int scratch_for_stream(hipStream_t stream, void** ptr) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (stream != nullptr) {
        hipDevice_t sdev = 0;
        e = hipStreamGetDevice(stream, &sdev);
        if (e != hipSuccess) return hip_fail(e, "hipStreamGetDevice");
        if (sdev != dev)
            return fail(CA_ERR_INVALID, "the stream belongs to device %d but device %d is current", (int)sdev, dev);
    }
    if (dev < 0 || dev >= kMaxDevices) return fail(CA_ERR_LIMIT, "device %d beyond the %d supported", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return CA_OK;
}

}  // namespace

extern "C" {

int ca_abi_version(void) { return CA_ABI_VERSION; }

const char* ca_last_error(void) { return g_last_error.c_str(); }

int ca_cache_fill(const ca_dims* dims, const ca_seq_layout* k_new, const ca_seq_layout* v_new,
                  const ca_kv_layout* k_cache, const ca_kv_layout* v_cache,
                  const int32_t* past_blocks_host, float* kmean, const float* gate_wk,
                  const float* rope_cos, const float* rope_sin, int64_t rope_rows, float* kgate,
                  void* stream) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0, rc;
    if ((rc = check_dims(dims, past_blocks_host, &s, &pb, &max_nkb)) != CA_OK) return rc;
    ca::SeqAddr kn{}, vn{};
    ca::KvAddr kc{}, vc{};
    if ((rc = check_seq(k_new, "k_new", &kn)) != CA_OK) return rc;
    const bool copy = k_cache != nullptr || v_cache != nullptr;
    if (copy) {
        if ((rc = check_seq(v_new, "v_new", &vn)) != CA_OK) return rc;
        if ((rc = check_kv(k_cache, "k_cache", max_nkb, &kc)) != CA_OK) return rc;
        if ((rc = check_kv(v_cache, "v_cache", max_nkb, &vc)) != CA_OK) return rc;
    } else if (kmean == nullptr && gate_wk == nullptr) {
        return fail(CA_ERR_INVALID, "nothing to do: no cache and no summary output");
    }
    if (kmean != nullptr && !aligned16(kmean)) return fail(CA_ERR_INVALID, "kmean misaligned");
    if (gate_wk != nullptr) {
        if (kgate == nullptr) return fail(CA_ERR_INVALID, "gate_wk given without kgate");
        if ((rc = check_rope(rope_cos, rope_sin, rope_rows, max_nkb)) != CA_OK) return rc;
    }
    hipError_t e = ca::launch_cache_fill(s, kn, vn, kc, vc, pb, kmean, gate_wk, rope_cos, rope_sin,
                                         kgate, CA_POOL_AVG, 1, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "cache_fill launch");
    return ok();
}

int ca_gate_key_summaries(const ca_dims* dims, const ca_seq_layout* k_new, const int32_t* past_blocks_host,
                          int32_t pools, const float* gate_wk, int32_t gate_heads, const float* rope_cos,
                          const float* rope_sin, int64_t rope_rows, float* kgate, void* stream) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0, rc;
    if ((rc = check_dims(dims, past_blocks_host, &s, &pb, &max_nkb)) != CA_OK) return rc;
    ca::SeqAddr kn{};
    if ((rc = check_seq(k_new, "k_new", &kn)) != CA_OK) return rc;
    if ((rc = check_pools(pools)) != CA_OK) return rc;
    if (gate_wk == nullptr || kgate == nullptr) return fail(CA_ERR_INVALID, "gate_wk and kgate are required");
    if (!aligned4(gate_wk) || !aligned4(kgate)) return fail(CA_ERR_INVALID, "gate_wk / kgate misaligned");
    if (gate_heads != s.Hkv && gate_heads != s.Hq)
        return fail(CA_ERR_INVALID, "gate_heads=%d must be num_kv_heads=%d or num_q_heads=%d", gate_heads, s.Hkv,
                    s.Hq);
    if ((rc = check_rope(rope_cos, rope_sin, rope_rows, max_nkb)) != CA_OK) return rc;
    const ca::KvAddr none{};
    hipError_t e = ca::launch_cache_fill(s, kn, kn, none, none, pb, nullptr, gate_wk, rope_cos, rope_sin, kgate,
                                         pools, gate_heads / s.Hkv, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "gate_key_summaries launch");
    return ok();
}

int ca_gate_query_summaries(const ca_dims* dims, const ca_seq_layout* q, const int32_t* past_blocks_host,
                            int32_t pools, const float* gate_wq, int32_t gate_heads, const float* rope_cos,
                            const float* rope_sin, int64_t rope_rows, float* qhat, void* stream) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0, rc;
    if ((rc = check_dims(dims, past_blocks_host, &s, &pb, &max_nkb)) != CA_OK) return rc;
    ca::SeqAddr qa;
    if ((rc = check_seq(q, "q", &qa)) != CA_OK) return rc;
    if ((rc = check_pools(pools)) != CA_OK) return rc;
    if (qhat == nullptr || !aligned4(qhat)) return fail(CA_ERR_INVALID, "qhat is NULL or misaligned");
    const bool single = pools == CA_POOL_MAX || pools == CA_POOL_MIN || pools == CA_POOL_AVG;
    if (gate_wq == nullptr) {
        if (!single) return fail(CA_ERR_INVALID, "more than one query pool needs a projection (gate_wq)");
        if (gate_heads != s.Hq)
            return fail(CA_ERR_INVALID, "gate_heads=%d: unprojected query summaries have num_q_heads=%d heads",
                        gate_heads, s.Hq);
    } else {
        if (!aligned4(gate_wq)) return fail(CA_ERR_INVALID, "gate_wq misaligned");
        if (gate_heads != s.Hq && gate_heads != s.Hkv)
            return fail(CA_ERR_INVALID, "gate_heads=%d must be num_q_heads=%d or num_kv_heads=%d", gate_heads, s.Hq,
                        s.Hkv);
    }
    // the block RoPE applies with or without a projection (attn_gate.py:138-171)
    if ((rc = check_rope(rope_cos, rope_sin, rope_rows, max_nkb)) != CA_OK) return rc;
    const bool kv_aware = gate_wq != nullptr && gate_heads == s.Hkv && s.Hq != s.Hkv;
    hipError_t e = ca::launch_pool_query(s, qa, pb, gate_wq, rope_cos, rope_sin, qhat, pools, kv_aware,
                                         static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "gate_query_summaries launch");
    return ok();
}

int ca_cache_fill_pool_query(const ca_dims* dims, const ca_seq_layout* k_new, const ca_seq_layout* v_new,
                             const ca_kv_layout* k_cache, const ca_kv_layout* v_cache,
                             const int32_t* past_blocks_host, float* kmean, const ca_seq_layout* q, float* qhat,
                             void* stream) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0, rc;
    if ((rc = check_dims(dims, past_blocks_host, &s, &pb, &max_nkb)) != CA_OK) return rc;
    ca::SeqAddr kn{}, vn{}, qa{};
    ca::KvAddr kc{}, vc{};
    if ((rc = check_seq(k_new, "k_new", &kn)) != CA_OK) return rc;
    if ((rc = check_seq(v_new, "v_new", &vn)) != CA_OK) return rc;
    if ((rc = check_kv(k_cache, "k_cache", max_nkb, &kc)) != CA_OK) return rc;
    if ((rc = check_kv(v_cache, "v_cache", max_nkb, &vc)) != CA_OK) return rc;
    if ((rc = check_seq(q, "q", &qa)) != CA_OK) return rc;
    if (kmean == nullptr || qhat == nullptr) return fail(CA_ERR_INVALID, "kmean and qhat are required");
    if (!aligned16(kmean)) return fail(CA_ERR_INVALID, "kmean misaligned");
    hipError_t e = ca::launch_chunk_summaries(s, kn, vn, kc, vc, pb, kmean, qa, qhat, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "cache_fill_pool_query launch");
    return ok();
}

int ca_pool_query(const ca_dims* dims, const ca_seq_layout* q, const int32_t* past_blocks_host,
                  const float* gate_wq, const float* rope_cos, const float* rope_sin,
                  int64_t rope_rows, float* qhat, void* stream) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0, rc;
    if ((rc = check_dims(dims, past_blocks_host, &s, &pb, &max_nkb)) != CA_OK) return rc;
    ca::SeqAddr qa;
    if ((rc = check_seq(q, "q", &qa)) != CA_OK) return rc;
    if (qhat == nullptr) return fail(CA_ERR_INVALID, "qhat is NULL");
    if (gate_wq != nullptr && (rc = check_rope(rope_cos, rope_sin, rope_rows, max_nkb)) != CA_OK) return rc;
    hipError_t e = ca::launch_pool_query(s, qa, pb, gate_wq, gate_wq ? rope_cos : nullptr,
                                         gate_wq ? rope_sin : nullptr, qhat, CA_POOL_AVG, false,
                                         static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "pool_query launch");
    return ok();
}

int ca_pair_block_summaries(const float* src, int64_t src_stride, float* dst, int64_t dst_stride, int64_t rows,
                            int32_t n_blocks, int32_t last_tokens, void* stream) {
    if (src == nullptr || dst == nullptr) return fail(CA_ERR_INVALID, "src and dst are required");
    if (!aligned16(src) || !aligned16(dst)) return fail(CA_ERR_INVALID, "src and dst must be 16-byte aligned");
    if (rows < 1 || n_blocks < 1) return fail(CA_ERR_INVALID, "rows=%lld and n_blocks=%d must be positive",
                                              (long long)rows, n_blocks);
    if (last_tokens < 1 || last_tokens > CA_BLOCK)
        return fail(CA_ERR_INVALID, "last_tokens=%d outside [1, %d]", last_tokens, CA_BLOCK);
    const int npairs = (n_blocks + 1) / 2;
    if (src_stride < n_blocks || dst_stride < npairs)
        return fail(CA_ERR_INVALID, "row strides (%lld, %lld blocks) below (%d, %d)", (long long)src_stride,
                    (long long)dst_stride, n_blocks, npairs);
    if (rows * npairs > ((int64_t)1 << 36)) return fail(CA_ERR_LIMIT, "too many rows");
    hipError_t e = ca::launch_pair_summaries(src, src_stride, dst, dst_stride, rows, n_blocks, last_tokens,
                                             static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "pair_summaries launch");
    return ok();
}

int ca_score_select(const ca_dims* dims, const float* qhat, const float* khat, float scale,
                    const ca_select_rule* rule, const int32_t* past_blocks_host, uint32_t* rowmask,
                    float* scores, void* stream) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0, rc;
    if ((rc = check_dims(dims, past_blocks_host, &s, &pb, &max_nkb)) != CA_OK) return rc;
    if ((rc = check_rule(rule)) != CA_OK) return rc;
    if (qhat == nullptr || khat == nullptr || rowmask == nullptr || scores == nullptr)
        return fail(CA_ERR_INVALID, "qhat, khat, rowmask and scores are required");
    if (!aligned16(khat) || !aligned16(qhat)) return fail(CA_ERR_INVALID, "qhat and khat must be 16-byte aligned");
    if (ca::score_select_lds_bytes(s, true) > kMaxLds)
        return fail(CA_ERR_LIMIT, "group %d x kv_cap %d scores do not fit in LDS", s.G, s.cap);
    hipError_t e = ca::launch_score_select(s, qhat, khat, scale, nullptr, 0, 0, 0, 0, *rule, pb, rowmask,
                                           scores, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "score_select launch");
    return ok();
}

int ca_score_token_mass(const ca_dims* dims, const ca_seq_layout* q, const float* khat, int64_t khat_stride,
                        int32_t block_size, float scale, const int32_t* past_blocks_host, float* scores,
                        void* stream) {
    if (dims == nullptr || past_blocks_host == nullptr) return fail(CA_ERR_INVALID, "dims and past_blocks are required");
    if (block_size != 64 && block_size != 128) return fail(CA_ERR_INVALID, "block_size=%d (64 or 128)", block_size);
    // dims count block_size blocks: the 64-token shape checks run on the same numbers with the
    // chunk's blocks counted in block_size units
    ca_dims d64 = *dims;
    const int qb = (dims->q_len + block_size - 1) / block_size;
    d64.q_len = qb * CA_BLOCK;  // Qb = qb in the shape checks below
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0, rc;
    if ((rc = check_dims(&d64, past_blocks_host, &s, &pb, &max_nkb)) != CA_OK) return rc;
    s.Lq = dims->q_len;
    ca::SeqAddr qa;
    if ((rc = check_seq(q, "q", &qa)) != CA_OK) return rc;
    if (khat == nullptr || scores == nullptr) return fail(CA_ERR_INVALID, "khat and scores are required");
    if (!aligned16(khat) || !aligned16(scores)) return fail(CA_ERR_INVALID, "khat and scores must be 16-byte aligned");
    if (khat_stride < max_nkb)
        return fail(CA_ERR_INVALID, "khat_stride=%lld < key blocks per row %d", (long long)khat_stride, max_nkb);
    for (int b = 0; b < s.B; ++b)
        if ((int64_t)past_blocks_host[b] * block_size > ((int64_t)1 << 30))
            return fail(CA_ERR_LIMIT, "past_blocks[%d]=%d: positions beyond 2^30 tokens", b, past_blocks_host[b]);
    if (ca::token_mass_lds_bytes(s, block_size) > kMaxLds) return fail(CA_ERR_LIMIT, "kv_cap=%d too large", s.cap);
    hipError_t e = ca::launch_token_mass(s, qa, khat, khat_stride, block_size, scale, pb, scores,
                                         static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "score_token_mass launch");
    return ok();
}

int ca_select_scores(const ca_dims* dims, const void* scores, int32_t dtype, int64_t stride_b,
                     int64_t stride_h, int64_t stride_q, const ca_select_rule* rule,
                     const int32_t* past_blocks_host, uint32_t* rowmask, void* stream) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0, rc;
    if ((rc = check_dims(dims, past_blocks_host, &s, &pb, &max_nkb)) != CA_OK) return rc;
    if ((rc = check_rule(rule)) != CA_OK) return rc;
    if (scores == nullptr || rowmask == nullptr) return fail(CA_ERR_INVALID, "scores and rowmask are required");
    if (dtype != 0 && dtype != 1) return fail(CA_ERR_INVALID, "dtype=%d (0 = fp32, 1 = bf16)", dtype);
    if (stride_b < 0 || stride_h < 0 || stride_q < 0) return fail(CA_ERR_INVALID, "negative score stride");
    if (ca::score_select_lds_bytes(s, false) > kMaxLds)
        return fail(CA_ERR_LIMIT, "group %d x kv_cap %d scores do not fit in LDS", s.G, s.cap);
    hipError_t e = ca::launch_score_select(s, nullptr, nullptr, 0.0f, scores, dtype, stride_b, stride_h,
                                           stride_q, *rule, pb, rowmask, nullptr,
                                           static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "select_scores launch");
    return ok();
}

int ca_union_compact(const ca_dims* dims, const uint32_t* rowmask, int32_t last_n_block,
                     const int32_t* past_blocks_host, uint8_t* keep_block, uint8_t* keep_kv,
                     int32_t* table, int64_t table_stride, int32_t* counts, void* stream) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0, rc;
    if ((rc = check_dims(dims, past_blocks_host, &s, &pb, &max_nkb)) != CA_OK) return rc;
    if (rowmask == nullptr || table == nullptr || counts == nullptr)
        return fail(CA_ERR_INVALID, "rowmask, table and counts are required");
    if (table_stride < s.cap) return fail(CA_ERR_INVALID, "table_stride=%lld < kv_cap=%d", (long long)table_stride, s.cap);
    if (ca::union_lds_bytes(s) > kMaxLds) return fail(CA_ERR_LIMIT, "kv_cap too large");
    hipError_t e = ca::launch_union_compact(s, rowmask, last_n_block, nullptr, pb, keep_block, keep_kv, table,
                                            table_stride, counts, false, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "union_compact launch");
    return ok();
}

int ca_compact_keep_kv(const ca_dims* dims, const uint8_t* keep_kv, const int32_t* past_blocks_host,
                       int32_t* table, int64_t table_stride, int32_t* counts, void* stream) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0, rc;
    if ((rc = check_dims(dims, past_blocks_host, &s, &pb, &max_nkb)) != CA_OK) return rc;
    if (keep_kv == nullptr || table == nullptr || counts == nullptr)
        return fail(CA_ERR_INVALID, "keep_kv, table and counts are required");
    if (table_stride < s.cap) return fail(CA_ERR_INVALID, "table_stride=%lld < kv_cap=%d", (long long)table_stride, s.cap);
    if (ca::union_lds_bytes(s) > kMaxLds) return fail(CA_ERR_LIMIT, "kv_cap too large");
    hipError_t e = ca::launch_union_compact(s, nullptr, 0, keep_kv, pb, nullptr, nullptr, table, table_stride,
                                            counts, false, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "compact_keep_kv launch");
    return ok();
}

int ca_dense_table(const ca_dims* dims, const int32_t* past_blocks_host, int32_t* table,
                   int64_t table_stride, int32_t* counts, void* stream) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0, rc;
    if ((rc = check_dims(dims, past_blocks_host, &s, &pb, &max_nkb)) != CA_OK) return rc;
    if (table == nullptr || counts == nullptr) return fail(CA_ERR_INVALID, "table and counts are required");
    if (table_stride < s.cap) return fail(CA_ERR_INVALID, "table_stride=%lld < kv_cap=%d", (long long)table_stride, s.cap);
    if (ca::union_lds_bytes(s) > kMaxLds) return fail(CA_ERR_LIMIT, "kv_cap too large");
    hipError_t e = ca::launch_union_compact(s, nullptr, 0, nullptr, pb, nullptr, nullptr, table, table_stride,
                                            counts, true, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "dense_table launch");
    return ok();
}

int ca_table_to_csr(const ca_dims* dims, const int32_t* table, int64_t table_stride, const int32_t* counts,
                    int32_t* kv_indptr, int32_t* kv_indices, int64_t indices_capacity, int32_t* kv_last_page_len,
                    void* stream) {
    if (dims == nullptr) return fail(CA_ERR_INVALID, "dims is NULL");
    if (dims->batch < 1 || dims->num_kv_heads < 1 || dims->kv_cap < 1)
        return fail(CA_ERR_INVALID, "batch, num_kv_heads and kv_cap must be positive");
    const int64_t rows = (int64_t)dims->batch * dims->num_kv_heads;
    if (rows > ca::kCsrRowsMax) return fail(CA_ERR_LIMIT, "rows=%lld > %d", (long long)rows, ca::kCsrRowsMax);
    if ((int64_t)dims->kv_cap * rows >= ((int64_t)1 << 31))
        return fail(CA_ERR_LIMIT, "rows * kv_cap must stay below 2^31 (int32 page ids)");
    if (table == nullptr || counts == nullptr || kv_indptr == nullptr || kv_indices == nullptr)
        return fail(CA_ERR_INVALID, "table, counts, kv_indptr and kv_indices are required");
    if (table_stride < dims->kv_cap)
        return fail(CA_ERR_INVALID, "table_stride=%lld < kv_cap=%d", (long long)table_stride, dims->kv_cap);
    if (indices_capacity < rows * dims->kv_cap)
        return fail(CA_ERR_INVALID, "indices_capacity=%lld < rows * kv_cap=%lld (the counts are not known on the host)",
                    (long long)indices_capacity, (long long)(rows * dims->kv_cap));
    hipError_t e = ca::launch_table_csr(table, table_stride, counts, static_cast<int>(rows), dims->kv_cap, kv_indptr,
                                        kv_indices, kv_last_page_len, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "table_to_csr launch");
    return ok();
}

int32_t ca_attn_pick_splits(const ca_dims* dims, const int32_t* past_blocks_host) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0;
    if (check_dims(dims, past_blocks_host, &s, &pb, &max_nkb) != CA_OK) return -1;
    return ca::attn_pick_splits(s, pb, nullptr);
}

int64_t ca_attn_workspace_size(const ca_dims* dims, const int32_t* past_blocks_host, int32_t num_splits) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0;
    if (check_dims(dims, past_blocks_host, &s, &pb, &max_nkb) != CA_OK) return -1;
    if (num_splits == 0) num_splits = ca::attn_pick_splits(s, pb, nullptr);
    if (num_splits < 1 || num_splits > ca::kMaxPrefillSplits)
        return fail(CA_ERR_INVALID, "num_splits=%d outside [0, %d]", num_splits, ca::kMaxPrefillSplits);
    return ca::attn_workspace_bytes(s, num_splits);
}

int ca_attn_fwd(const ca_dims* dims, const ca_seq_layout* q, const ca_kv_layout* k,
                const ca_kv_layout* v, const int32_t* table, int64_t table_stride,
                const int32_t* counts, const int32_t* past_blocks_host, float scale,
                const ca_seq_layout* out, float* lse, int32_t num_splits, void* workspace,
                int64_t workspace_bytes, void* stream) {
    ca::AttnArgs a;
    int max_nkb = 0, rc;
    if ((rc = check_dims(dims, past_blocks_host, &a.s, &a.pb, &max_nkb)) != CA_OK) return rc;
    if ((rc = check_seq(q, "q", &a.q)) != CA_OK) return rc;
    if ((rc = check_seq(out, "out", &a.out)) != CA_OK) return rc;
    if ((rc = check_kv(k, "k", max_nkb, &a.k)) != CA_OK) return rc;
    if ((rc = check_kv(v, "v", max_nkb, &a.v)) != CA_OK) return rc;
    if (table == nullptr || counts == nullptr) return fail(CA_ERR_INVALID, "table and counts are required");
    if (table_stride < a.s.cap) return fail(CA_ERR_INVALID, "table_stride=%lld < kv_cap=%d", (long long)table_stride, a.s.cap);
    if (!(scale > 0.0f)) return fail(CA_ERR_INVALID, "scale must be positive");
    if ((int64_t)a.s.Lq * a.s.G > (int64_t)1 << 24) return fail(CA_ERR_LIMIT, "q_len * group too large");
    if (num_splits < 0 || num_splits > ca::kMaxPrefillSplits)
        return fail(CA_ERR_INVALID, "num_splits=%d outside [0, %d]", num_splits, ca::kMaxPrefillSplits);
    const int max_splits = num_splits == 0 ? ca::attn_pick_splits(a.s, a.pb, nullptr) : num_splits;
    const int64_t need = ca::attn_workspace_bytes(a.s, max_splits);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)))
        return fail(CA_ERR_WORKSPACE, "num_splits=%d needs a 16-byte aligned workspace of %lld bytes (got %lld)",
                    num_splits, (long long)need, (long long)workspace_bytes);
    a.table = table;
    a.table_stride = table_stride;
    a.counts = counts;
    a.scale = scale;
    a.lse = lse;
    a.num_splits = num_splits;
    a.workspace = workspace;
    a.kv_len = nullptr;
    hipError_t e = ca::launch_attn(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "attn launch");
    return ok();
}

int ca_attn_fwd_noalloc(const ca_dims* dims, const ca_seq_layout* q, const ca_kv_layout* k,
                        const ca_kv_layout* v, const int32_t* table, int64_t table_stride,
                        const int32_t* counts, const int32_t* past_blocks_host, float scale,
                        const ca_seq_layout* out, float* lse, int32_t num_splits, void* stream) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0, rc;
    if ((rc = check_dims(dims, past_blocks_host, &s, &pb, &max_nkb)) != CA_OK) return rc;
    if (num_splits < 0 || num_splits > ca::kMaxPrefillSplits)
        return fail(CA_ERR_INVALID, "num_splits=%d outside [0, %d]", num_splits, ca::kMaxPrefillSplits);
    // num_splits = 0 passes through when the automatic count's partials fit the library's
    // scratch array (ca_attn_fwd then plans exactly as for num_splits = 0, including the ragged
    // launch's split-or-unsplit choice); otherwise the count is lowered until they fit and
    // forced
    int splits = num_splits;
    int forward = num_splits;
    if (splits == 0) {
        splits = ca::attn_pick_splits(s, pb, nullptr);
        if (ca::attn_workspace_bytes(s, splits) > (int64_t)CA_STATIC_SCRATCH_BYTES) {
            while (splits > 1 && ca::attn_workspace_bytes(s, splits) > (int64_t)CA_STATIC_SCRATCH_BYTES) --splits;
            forward = splits;
        }
    }
    const int64_t need = ca::attn_workspace_bytes(s, splits);
    if (need > (int64_t)CA_STATIC_SCRATCH_BYTES)
        return fail(CA_ERR_LIMIT, "num_splits=%d needs %lld bytes of split partials; the allocation-free entry "
                    "holds at most %lld (CA_STATIC_SCRATCH_BYTES)", splits, (long long)need,
                    (long long)CA_STATIC_SCRATCH_BYTES);
    void* ws = nullptr;
    if (need > 0 && (rc = scratch_for_stream(static_cast<hipStream_t>(stream), &ws)) != CA_OK) return rc;
    return ca_attn_fwd(dims, q, k, v, table, table_stride, counts, past_blocks_host, scale, out, lse, forward, ws,
                       need, stream);
}

int64_t ca_attn_decode_workspace_size(const ca_dims* dims, const int32_t* kv_len_host, int32_t num_splits) {
    ca::Shape s;
    ca::PastBlocks pb;
    int max_nkb = 0;
    if (check_decode_dims(dims, kv_len_host, &s, &pb, &max_nkb) != CA_OK) return -1;
    if (num_splits == 0) num_splits = ca::attn_pick_splits(s, pb, kv_len_host);
    if (num_splits < 1 || num_splits > ca::kMaxDecodeSplits)
        return fail(CA_ERR_INVALID, "num_splits=%d outside [0, %d]", num_splits, ca::kMaxDecodeSplits);
    return ca::attn_workspace_bytes(s, num_splits);
}

int ca_attn_decode(const ca_dims* dims, const ca_seq_layout* q, const ca_kv_layout* k,
                   const ca_kv_layout* v, const int32_t* kv_len_host, float scale,
                   const ca_seq_layout* out, float* lse, int32_t num_splits, void* workspace,
                   int64_t workspace_bytes, void* stream) {
    ca::AttnArgs a;
    int max_nkb = 0, rc;
    if ((rc = check_decode_dims(dims, kv_len_host, &a.s, &a.pb, &max_nkb)) != CA_OK) return rc;
    if ((rc = check_seq(q, "q", &a.q)) != CA_OK) return rc;
    if ((rc = check_seq(out, "out", &a.out)) != CA_OK) return rc;
    if ((rc = check_kv(k, "k", max_nkb, &a.k)) != CA_OK) return rc;
    if ((rc = check_kv(v, "v", max_nkb, &a.v)) != CA_OK) return rc;
    if (!(scale > 0.0f)) return fail(CA_ERR_INVALID, "scale must be positive");
    if (num_splits < 0 || num_splits > ca::kMaxDecodeSplits)
        return fail(CA_ERR_INVALID, "num_splits=%d outside [0, %d]", num_splits, ca::kMaxDecodeSplits);
    const int max_splits = num_splits == 0 ? ca::attn_pick_splits(a.s, a.pb, kv_len_host) : num_splits;
    const int64_t need = ca::attn_workspace_bytes(a.s, max_splits);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)))
        return fail(CA_ERR_WORKSPACE, "num_splits=%d needs a 16-byte aligned workspace of %lld bytes (got %lld)",
                    num_splits, (long long)need, (long long)workspace_bytes);
    a.table = nullptr;
    a.table_stride = 0;
    a.counts = nullptr;
    a.scale = scale;
    a.lse = lse;
    a.num_splits = num_splits;
    a.workspace = workspace;
    a.kv_len = kv_len_host;
    hipError_t e = ca::launch_attn(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "attn decode launch");
    return ok();
}

}  // extern "C"

// ---------------------------------------------------------------------------------------
// Model plumbing: fused element-wise kernels of the Llama integration.

int ca_rope_apply(const ca_seq_layout* x, const ca_seq_layout* y, int32_t batch, int32_t len, int32_t heads,
                  const float* cos, const float* sin, void* stream) {
    ca::SeqAddr xa, ya;
    int rc;
    if ((rc = check_seq(x, "x", &xa)) != CA_OK) return rc;
    if ((rc = check_seq(y, "y", &ya)) != CA_OK) return rc;
    if (batch < 1 || len < 1 || heads < 1) return fail(CA_ERR_INVALID, "batch, len and heads must be positive");
    if ((int64_t)batch * len >= ((int64_t)1 << 31) || heads > 65535)
        return fail(CA_ERR_LIMIT, "batch * len must be below 2^31 and heads at most 65535");
    if (cos == nullptr || sin == nullptr) return fail(CA_ERR_INVALID, "cos and sin are required");
    if (!aligned16(cos) || !aligned16(sin)) return fail(CA_ERR_INVALID, "cos and sin must be 16-byte aligned");
    hipError_t e = ca::launch_rope(xa, ya, cos, sin, batch, len, heads, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "rope launch");
    return ok();
}

int ca_rmsnorm(const uint16_t* x, int64_t x_stride, const uint16_t* residual, int64_t r_stride, uint16_t* sum_out,
               int64_t s_stride, const uint16_t* w, uint16_t* y, int64_t y_stride, int64_t rows, int32_t n, float eps,
               void* stream) {
    if (x == nullptr || w == nullptr || y == nullptr) return fail(CA_ERR_INVALID, "x, w and y are required");
    if (!aligned16(x) || !aligned16(w) || !aligned16(y)) return fail(CA_ERR_INVALID, "x, w and y must be 16-byte aligned");
    if (n < 8 || n % 8 || x_stride % 8 || y_stride % 8 || x_stride < n || y_stride < n)
        return fail(CA_ERR_INVALID, "n=%d must be a positive multiple of 8 and the row strides multiples of 8 >= n", n);
    if ((residual == nullptr) != (sum_out == nullptr))
        return fail(CA_ERR_INVALID, "residual and sum_out are given together or not at all");
    if (residual != nullptr) {
        if (!aligned16(residual) || !aligned16(sum_out))
            return fail(CA_ERR_INVALID, "residual and sum_out must be 16-byte aligned");
        if (r_stride % 8 || s_stride % 8 || r_stride < n || s_stride < n)
            return fail(CA_ERR_INVALID, "residual / sum_out row strides must be multiples of 8 >= n");
    }
    if (rows < 0 || rows >= ((int64_t)1 << 31)) return fail(CA_ERR_LIMIT, "rows=%lld outside [0, 2^31)", (long long)rows);
    if (!(eps >= 0.0f)) return fail(CA_ERR_INVALID, "eps must be >= 0");
    if (rows == 0) return ok();
    hipError_t e = ca::launch_rmsnorm(x, x_stride, residual, r_stride, sum_out, s_stride, w, y, y_stride, rows, n, eps,
                                      static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "rmsnorm launch");
    return ok();
}

int ca_swiglu(const uint16_t* gate, int64_t g_stride, const uint16_t* up, int64_t u_stride, uint16_t* y,
              int64_t y_stride, int64_t rows, int32_t n, void* stream) {
    if (gate == nullptr || up == nullptr || y == nullptr) return fail(CA_ERR_INVALID, "gate, up and y are required");
    if (!aligned16(gate) || !aligned16(up) || !aligned16(y))
        return fail(CA_ERR_INVALID, "gate, up and y must be 16-byte aligned");
    if (n < 8 || n % 8 || g_stride % 8 || u_stride % 8 || y_stride % 8 || g_stride < n || u_stride < n || y_stride < n)
        return fail(CA_ERR_INVALID, "n=%d must be a positive multiple of 8 and the row strides multiples of 8 >= n", n);
    if (rows < 0 || rows * (n / 8) >= ((int64_t)1 << 38)) return fail(CA_ERR_LIMIT, "too many elements");
    if (rows == 0) return ok();
    hipError_t e = ca::launch_swiglu(gate, g_stride, up, u_stride, y, y_stride, rows, n, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "swiglu launch");
    return ok();
}
