// Indexed attention prefill over selected KV blocks: bf16 MFMA (gfx950
// v_mfma_f32_32x32x16_bf16), online softmax, K/V blocks read through the block table.
//
// Reference semantics: flash_attn_with_kvcache / FlashInfer paged prefill as driven by
// compact_attn/kernels/varlen/indexed_dense_prefill_varlen.py:1473-1613 and
// compact_attn/kernels/varlen/flashinfer_zero_copy_prefill.py:1139-1353 (GQA-packed rows,
// bottom-right causal), restated without a gather in
// compact_attn/kernels/varlen/indexed_dense_prefill_direct_triton.py:91-241.
//
// Work decomposition
//  - The G query heads of a KV group share the group's block table, so a KV row
//    (request, kv head) owns Lq*G "packed" query rows r = t*G + g (token t, head g).
//  - A workgroup (8 waves, one per CU) takes 256 packed rows; each wave keeps 32 rows (one
//    32x32 MFMA tile) for the whole KV loop: Q in VGPRs, O^T in accumulators.  Each SIMD
//    runs two waves whose softmax and MFMA phases overlap; a wave raises its issue
//    priority while it feeds the S^T MFMAs.
//  - Scores are computed transposed, S^T = K Q^T (A = K from LDS, B = Q from VGPRs), so the
//    softmax output lands in exactly the VGPR layout the second product's B operand needs:
//    O^T += V^T P^T (A = V^T from LDS).  Inside each 32-key S^T tile the A-row -> key map
//    swaps bits 2 and 3 of the row index, which makes every lane's 8 P values 8 consecutive
//    keys.
//  - K and V blocks go from HBM to LDS by LDS-DMA buffer loads (no staging registers),
//    row-major with XOR swizzles that keep the fragment reads free of bank conflicts.  V^T
//    fragments are read with the gfx950 transposing LDS read (ds_read_b64_tr_b16), two
//    per MFMA.
//  - Four LDS stages: the DMA of the next three blocks is in flight while the current
//    block is computed, and a step waits only for the block after it.  Optional split of
//    each row's block list (split-KV) with an LSE merge.
//  - Workgroup ids are remapped so consecutive work items (same KV row) share an XCD and
//    its L2.

#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

constexpr int kNW = 8;     // waves per workgroup (32 packed query rows each)
constexpr int kStages = 4;  // LDS stages (K + V of one block each): 128 KB per workgroup
constexpr int kBM = 32 * kNW;        // packed query rows per workgroup
constexpr int kKBytes = 64 * 256;  // K rows of one block in LDS (swizzled, unpadded)
constexpr int kVBytes = 64 * 256;  // V rows of one block in LDS (swizzled, unpadded)
constexpr int kStageBytes = kKBytes + kVBytes;
constexpr float kRescale = 8.0f;      // lazy-rescale slack (log2 units)

struct AttnParams {
    Shape s;
    SeqAddr q;
    KvAddr k, v;
    const int32_t* table;
    int64_t table_stride;
    const int32_t* counts;
    PastBlocks pb;
    float scale_log2;  // softmax scale * log2(e)
    SeqAddr out;
    float* lse;
    int ntiles;       // packed-row tiles per KV row
    int rows_total;   // Lq * G
    int total_items;  // B*Hkv*ntiles*splits
    int per_xcd;      // ceil(total_items / 8)
    float* ws_o;      // [max splits][B*Hkv][rows_total][128]
    float* ws_lse;    // [max splits][B*Hkv][rows_total]  (log2 domain)
    // Ragged prefill whose row tiles fill 3/4 of the CUs: the kernel runs unsplit when every
    // row's selected count is within 1.5x of their mean (workgroup 0 records the choice
    // here for the merge); null otherwise
    int32_t* ws_unsplit;
    // K and V without page tables, 64-token blocks contiguous in token order (stride_blk =
    // 64 stride_tok) and every request's tokens within 2^31 bytes: the DMA addresses a block
    // through one buffer resource per KV row (the block's byte offset in the scalar offset),
    // whose range ends at the request's last token as the per-block resources do
    int row_res;
    int32_t qpos0[CA_MAX_BATCH];     // absolute position of each request's query row 0
    int32_t nkb[CA_MAX_BATCH];       // valid logical blocks of each request
    int32_t sp[CA_MAX_BATCH];        // splits of each request's block lists
    int32_t ioff[CA_MAX_BATCH + 1];  // first work item of each request (linear placement)
    int use_rows;                    // units placed per XCD (xoff / xrow / xlo / xcnt)
    int32_t xoff[9];
    uint16_t xrow[kPlanRows];
    uint8_t xlo[kPlanRows];
    uint8_t xcnt[kPlanRows];
};

__device__ __forceinline__ int swap23(int m) {
    return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1);
}

__device__ __forceinline__ lds_void_t* to_lds(const uint8_t* p) {
    return (lds_void_t*)(p);
}
__device__ __forceinline__ lds_i16x4_t* to_lds_v4(const uint8_t* p) {
    return (lds_i16x4_t*)(p);
}
// max(x, x of lane ^ 32): v_permlane32_swap hands each half the other half's values, so
// the max of its two outputs is the pair's max in every lane (no LDS round trip).
__device__ __forceinline__ float xor32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// max(x, x of lane ^ 16), the same way with v_permlane16_swap
__device__ __forceinline__ float xor16_max(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Wave-uniform reads of tables the kernel never writes (block ids, counts, page tables) go
// through the scalar data cache: s_load waits on lgkmcnt, so they do not queue behind the
// LDS-DMA loads in flight on vmcnt.
typedef const __attribute__((address_space(4))) int32_t const_i32_t;
__device__ __forceinline__ int32_t sload(const int32_t* p) {
    return *(const_i32_t*)p;
}
// Completes this wave's outstanding LDS-DMA loads (vector-memory counter).
__device__ __forceinline__ void wait_dma() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}


// NW waves per workgroup, 32 packed query rows per wave (one 32x32 MFMA row tile), so a
// workgroup owns BM = 32*NW rows.  Registers stay within 256 per lane, which lets two waves
// share a SIMD: one wave's softmax overlaps the other's MFMAs.  One 8-wave workgroup per
// CU (128 KB of LDS).
// kTab: block lists come from the per-row table (prefill); otherwise they are the identity
// 0 .. nkb-1 (dense decode).
template <int NW, bool kTab>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void attn_fwd_kernel(AttnParams p) {
    constexpr int BM = 32 * NW;
    __shared__ __attribute__((aligned(16))) uint8_t smem[kStages * kStageBytes];  // [stage]: K rows, then V rows

    // Ragged launches whose row tiles fill 3/4 of the CUs: one round of row tiles is enough
    // when the rows' selected counts are even, so the items of the other splits have nothing
    // to do.  Every workgroup derives the same choice from the counts (wave 0, the flag through
    // LDS before the stages are used; workgroup 0 records it for the merge).
    int unsplit = 0;
    if (kTab && p.ws_unsplit) {
        volatile int* flag = reinterpret_cast<volatile int*>(smem);
        if (threadIdx.x < 64) {
            const int rows = p.s.B * p.s.Hkv;
            int64_t sum = 0;
            int mx = 0;
            for (int r = threadIdx.x; r < rows; r += 64) {
                const int c = min(max(p.counts[r], 0), p.s.cap);
                sum += c;
                mx = max(mx, c);
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                sum += __shfl_xor(sum, o, 64);
                mx = max(mx, __shfl_xor(mx, o, 64));
            }
            if (threadIdx.x == 0) {
                const int even = 2 * (int64_t)mx * rows <= 3 * sum ? 1 : 0;  // max <= 1.5 x mean
                *flag = even;
                if (blockIdx.x == 0) *p.ws_unsplit = even;
            }
        }
        __syncthreads();
        // uniform by construction; readfirstlane tells the compiler, which keeps the block-id
        // and table reads that depend on it scalar (vector loads would wait behind the DMA)
        unsplit = __builtin_amdgcn_readfirstlane(*flag);
        __syncthreads();
    }

    // workgroup -> (XCD x, k-th work item of x) -> (KV row, row tile, split)
    const int L = blockIdx.x;
    const int x = L & 7;
    int k = L >> 3;
    const Shape& s = p.s;
    int row, b, split, tile;
    if (p.use_rows && kTab && unsplit) {
        // an unsplit launch takes the XCD's items split-major (its units are whole rows with
        // one split count): the items of split 0 of every unit first, so the working items are
        // dispatched first and the idle ones after them (interleaved, the idle items held the
        // working ones back: 510 vs 290 us on config 4); a split launch keeps the unit-major
        // order below, which runs a long row's items before a short row's
        const int i0 = p.xoff[x];
        const int per = (p.xoff[x + 1] - i0) * p.ntiles;  // items of one split on this XCD
        if (per == 0) return;
        const int sidx = k / per;
        const int kk = k - sidx * per;
        const int i = i0 + kk / p.ntiles;
        if (sidx >= p.xcnt[i]) return;
        row = p.xrow[i];
        b = row / s.Hkv;
        split = p.xlo[i] + sidx;
        tile = kk - (kk / p.ntiles) * p.ntiles;
    } else if (p.use_rows) {
        int i = p.xoff[x];
        const int iend = p.xoff[x + 1];
        for (; i < iend; ++i) {
            const int items = p.ntiles * p.xcnt[i];
            if (k < items) break;
            k -= items;
        }
        if (i >= iend) return;
        row = p.xrow[i];
        b = row / s.Hkv;
        split = p.xlo[i] + k % p.xcnt[i];
        tile = k / p.xcnt[i];
    } else {
        const int W = x * p.per_xcd + k;
        if (W >= p.total_items) return;
        b = 0;
        while (b + 1 < s.B && p.ioff[b + 1] <= W) ++b;
        const int per_row = p.ntiles * p.sp[b];
        row = b * s.Hkv + (W - p.ioff[b]) / per_row;
        const int local = (W - p.ioff[b]) % per_row;
        split = local % p.sp[b];
        tile = local / p.sp[b];
    }
    const int hk = row - b * s.Hkv;
    int nsplit = p.sp[b];
    if (unsplit) {
        if (split != 0) return;
        nsplit = 1;
    }
    const int G = s.G;
    const int qpos0 = p.qpos0[b];  // query row t sits at absolute position qpos0 + t
    const int nkb = p.nkb[b];      // valid logical block ids are [0, nkb)
    const int rows_total = p.rows_total;
    const int r0 = tile * BM;
    const int t_first = r0 / G;
    const int t_last = min(r0 + BM - 1, rows_total - 1) / G;

    // Table entries are clamped into [0, nkb) so a corrupt table cannot address outside the
    // KV tensors.
    const int32_t* tab = kTab ? p.table + (int64_t)row * p.table_stride : nullptr;
    auto block_id = [&](int e) { return kTab ? min(max(sload(tab + e), 0), nkb - 1) : e; };
    const int lim = (qpos0 + t_last) >> 6;  // last block the tile can see
    int n_vis;
    if (kTab) {
        n_vis = min(max(sload(p.counts + row), 0), s.cap);
        while (n_vis > 0 && sload(tab + n_vis - 1) > lim) --n_vis;
    } else {
        n_vis = min(nkb, lim + 1);
    }
    const int chunk = (n_vis + nsplit - 1) / nsplit;
    const int e0 = min(n_vis, split * chunk);
    const int e1 = min(n_vis, e0 + chunk);
    // entries at or after e_mask contain keys beyond the tile's first query position
    int e_mask = e1;
    while (e_mask > e0 && block_id(e_mask - 1) * 64 + 63 > qpos0 + t_first) --e_mask;

    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int l = tid & 63;
    const int h = l >> 5;
    const int n = l & 31;

    // ---- Q fragments (B operand of S^T = K Q^T) ----
    const int qrow = r0 + 32 * w + n;
    const bool qvalid = qrow < rows_total;
    const int qt = qvalid ? qrow / G : 0;
    const int qg = qvalid ? qrow - qt * G : 0;
    bf16x8_t qf[8];
    {
        const uint16_t* qp = p.q.data + b * p.q.sb + (int64_t)qt * p.q.st + (int64_t)(hk * G + qg) * p.q.sh + 8 * h;
#pragma unroll
        for (int ds = 0; ds < 8; ++ds) {
            if (qvalid) {
                qf[ds] = *reinterpret_cast<const bf16x8_t*>(qp + 16 * ds);
            } else {
                u32x4_t z = {0u, 0u, 0u, 0u};
                qf[ds] = __builtin_bit_cast(bf16x8_t, z);
            }
        }
    }
    const int qtok = qvalid ? qt : 0x3fffffff;

    f32x16_t oacc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j) oacc[dt][j] = 0.0f;
    float m_run = -__builtin_inff();
    float l_run = 0.0f;

    const uint16_t* kbase_row = p.k.data + b * p.k.sb + hk * p.k.sh;
    const uint16_t* vbase_row = p.v.data + b * p.v.sb + hk * p.v.sh;
    const int32_t* kpt = p.k.page_table ? p.k.page_table + (int64_t)row * p.k.pts : nullptr;
    const int32_t* vpt = p.v.page_table ? p.v.page_table + (int64_t)row * p.v.pts : nullptr;

    // ---- global -> LDS staging of one block (LDS DMA) ----
    // A block is 64 K rows and 64 V rows of 256 bytes.  Each wave issues 2 + 2 buffer loads
    // that write LDS directly (1 KB per instruction: lane L fills bytes 16L..16L+15 of the
    // instruction's 4 rows); the lane chooses which global 16-byte chunk lands there, which
    // applies the XOR swizzles.  Wave w moves rows 4w + 32i + L/16 (i = 0, 1), so a lane's
    // swizzle is the same for its two rows:
    //   K: 16-byte chunk c of row r sits at chunk c ^ (r & 15)    (conflict-free b128 reads)
    //   V: 16-byte chunk c of row r sits at chunk c ^ 4 (r & 3)   (conflict-free transposed reads)
    // 32-bit offsets inside a block (the host checks 64 * stride_tok < 2^30) on top of a
    // wave-uniform block base in the buffer resource.
    static_assert(NW == 8, "the staging split assumes eight waves");
    const int wu = __builtin_amdgcn_readfirstlane(w);
    const int st_row = 4 * wu + (l >> 4);
    const int kstok_b = static_cast<int>(p.k.stok) * 2;
    const int vstok_b = static_cast<int>(p.v.stok) * 2;
    const int k_goff = st_row * kstok_b + (((l & 15) ^ (st_row & 15)) * 16);
    const int v_goff = st_row * vstok_b + (((l & 15) ^ (4 * (st_row & 3))) * 16);
    // The request holds qpos0 + Lq tokens (kv_len in decode, whole blocks in prefill).  The
    // buffer range of a block ends after its last existing token, so the rows past kv_len of
    // a partial block read as zeros, whatever the cache holds there (masked keys get P = 0,
    // and 0 * V must not meet a non-finite V).  Row offsets go in the VGPR offset, which the
    // range check covers.
    const int kv_tokens = qpos0 + s.Lq;
    const __amdgpu_buffer_rsrc_t rk_row =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase_row), 0, kv_tokens * kstok_b, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv_row =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vbase_row), 0, kv_tokens * vstok_b, 0x00020000);
    const int kblk_b = 64 * kstok_b;
    const int vblk_b = 64 * vstok_b;
    auto issue_block = [&](int e, int stage) {
        const int kb = block_id(e);
        if (p.row_res) {
            uint8_t* kdst = smem + stage * kStageBytes + wu * 1024;
            uint8_t* vdst = kdst + kKBytes;
            // the block offset goes in the vector offset, which the range check covers (the
            // scalar offset is not checked)
            const int ko = k_goff + kb * kblk_b;
            const int vo = v_goff + kb * vblk_b;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rk_row, to_lds(kdst + i * 8192), 16, ko + i * 32 * kstok_b, 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rv_row, to_lds(vdst + i * 8192), 16, vo + i * 32 * vstok_b, 0, 0, 0);
            }
            return;
        }
        const int64_t kphys = kpt ? clamp_page(sload(kpt + kb), p.k.max_page) : kb;
        const int64_t vphys = vpt ? clamp_page(sload(vpt + kb), p.v.max_page) : kb;
        const int rows = min(kv_tokens - kb * 64, 64);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(kbase_row + kphys * p.k.sblk), 0, rows * kstok_b, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(vbase_row + vphys * p.v.sblk), 0, rows * vstok_b, 0x00020000);
        uint8_t* kdst = smem + stage * kStageBytes + wu * 1024;
        uint8_t* vdst = kdst + kKBytes;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, to_lds(kdst + i * 8192), 16, k_goff + i * 32 * kstok_b, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, to_lds(vdst + i * 8192), 16, v_goff + i * 32 * vstok_b, 0, 0, 0);
        }
    };

    const float sl2 = p.scale_log2;

    // One 64-key block: S^T = K Q^T (16 MFMAs), online softmax with lazy rescale, then
    // O^T += V^T P^T (16 MFMAs).  m_run only rises when a row's scaled block max exceeds it
    // by more than kRescale (log2 units); otherwise P = exp2(s - m_run) < 2^kRescale and the
    // accumulators keep their scale.
    // Fragment addresses.  K (A operand of S^T): lane row swap23(n) (+32 per 32-key half),
    // 16 bytes at d = 16 ds + 8 h.  V^T (A operand of O^T): each transposed b64 read gives
    // a lane 4 keys of one d column: lane l reads the 8 bytes at row 16 s4 + 8 h + 4 hh +
    // (l & 15) / 4, d = 32 dt + 16 ((l >> 4) & 1) + 4 (l & 3), which hands it keys
    // 16 s4 + 8 h + 4 hh + i (i = 0..3) of column d = 32 dt + n.  s4 and hh are immediates.
    const int k_r = swap23(n);
    int k_off[8];
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) k_off[ds] = k_r * 256 + (((2 * ds + h) ^ (k_r & 15)) * 16);
    const int v_rq = (l & 15) >> 2;
    const int v_x = 2 * ((l >> 4) & 1) + ((l & 3) >> 1);
    int v_off[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) v_off[dt] = (8 * h + v_rq) * 256 + (4 * (dt ^ v_rq) + v_x) * 16 + (l & 1) * 8;
    auto process = [&](int kb, const uint8_t* stage_base, bool masked) {
        const uint8_t* ks = stage_base;
        const uint8_t* vs = stage_base + kKBytes;
        f32x16_t sacc[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int j = 0; j < 16; ++j) sacc[kt][j] = 0.0f;
        // the two 32-key accumulators alternate so consecutive MFMAs are independent; the
        // K fragment reads run six ahead of the MFMAs (scheduling groups below)
        __builtin_amdgcn_s_setprio(1);
        {
            bf16x8_t kfr[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) kfr[i] = *reinterpret_cast<const bf16x8_t*>(ks + k_off[i >> 1] + (i & 1) * 8192);
#pragma unroll
            for (int i = 0; i < 16; ++i)
                sacc[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[i], qf[i >> 1], sacc[i & 1], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);  // 6 LDS reads
#pragma unroll
            for (int i = 0; i < 10; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
        }
        __builtin_amdgcn_s_setprio(0);
        if (masked) {
            // value j of half kt holds key kt*32 + swap23(8*(j/4) + 4*h + j%4)
            // = kt*32 + 8*h + key_off(j); visible iff kb*64 + key <= qpos0 + t
            const int vis = qpos0 + qtok - kb * 64 - 8 * h;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int key = kt * 32 + 16 * (j >> 3) + 4 * ((j >> 2) & 1) + (j & 3);
                    if (key > vis) sacc[kt][j] = -__builtin_inff();
                }
        }
        float mx = -__builtin_inff();
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int j = 0; j < 16; ++j) mx = fmaxf(mx, sacc[kt][j]);
        mx = xor32_max(mx) * sl2;
        float alpha = 1.0f;
        if (mx > m_run + kRescale) {
            alpha = __builtin_amdgcn_exp2f(m_run - mx);  // 0 when m_run = -inf
            m_run = mx;
            l_run *= alpha;
        }
        if (__ballot(alpha != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int j = 0; j < 16; ++j) oacc[dt][j] *= alpha;
        }
        const float m_use = m_run == -__builtin_inff() ? 0.0f : m_run;
        bf16x8_t pf[4];
        float rs = 0.0f;
        const bf16x2_t ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            f32x8_t pv8;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                pv8[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[s4 >> 1][8 * (s4 & 1) + i], sl2, -m_use));
            pf[s4] = __builtin_convertvector(pv8, bf16x8_t);
            // the normaliser sums the bf16-rounded weights the PV product uses
            rs = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf[s4], pf[s4], 0, 1), ones, rs, false);
            rs = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf[s4], pf[s4], 2, 3), ones, rs, false);
            rs = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf[s4], pf[s4], 4, 5), ones, rs, false);
            rs = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf[s4], pf[s4], 6, 7), ones, rs, false);
        }
        l_run += rs;  // this lane's half of the row; combined across lanes n, n+32 at the end
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(to_lds_v4(vs + v_off[dt] + s4 * 4096));
                const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(to_lds_v4(vs + v_off[dt] + s4 * 4096 + 1024));
                const bf16x8_t a = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf[s4], oacc[dt], 0, 0, 0);
            }
        }
    };

    // ---- KV loop: four LDS stages, DMA three blocks ahead ----
    const int nblk = e1 - e0;
    for (int i = 0; i < 3; ++i)
        if (i < nblk) issue_block(e0 + i, i);
    // block 0 must have landed (4 loads per block and wave)
    if (nblk > 2) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if (nblk > 1) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else wait_dma();
    __syncthreads();
    auto step = [&](int idx, bool masked) {
        if (idx + 3 < nblk) issue_block(e0 + idx + 3, (idx + 3) % kStages);
        process(block_id(e0 + idx), smem + (idx % kStages) * kStageBytes, masked);
        // block idx+1 must have landed; later blocks may stay in flight
        if (idx + 3 < nblk) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else if (idx + 2 < nblk) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        else wait_dma();
        __syncthreads();
    };
    int idx = 0;
    for (; idx < e_mask - e0; ++idx) step(idx, false);
    for (; idx < nblk; ++idx) step(idx, true);

    // ---- epilogue ----
    // lanes n and n + 32 hold different keys of the same row: their partial sums combine
    // here (both were rescaled by the same factors)
    l_run += __shfl_xor(l_run, 32, 64);
    if (qvalid) {
        const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
        const float lse2 = l_run > 0.0f ? m_run + __log2f(l_run) : -__builtin_inff();
        if (nsplit == 1) {
            const int hq = hk * G + qg;
            uint16_t* op = p.out.data + b * p.out.sb + (int64_t)qt * p.out.st + (int64_t)hq * p.out.sh;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int jq = 0; jq < 4; ++jq) {
                    const int d0 = dt * 32 + 8 * jq + 4 * h;
                    f32x4_t o4;
#pragma unroll
                    for (int i = 0; i < 4; ++i) o4[i] = oacc[dt][4 * jq + i] * inv;
                    *reinterpret_cast<bf16x4_t*>(op + d0) = __builtin_convertvector(o4, bf16x4_t);
                }
            if (p.lse && h == 0) p.lse[((int64_t)b * s.Hq + hq) * s.Lq + qt] = lse2 * 0.69314718055994531f;
        } else {
            const int64_t prow = ((int64_t)split * (s.B * s.Hkv) + row) * rows_total + qrow;
            float* wo = p.ws_o + prow * 128;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int jq = 0; jq < 4; ++jq) {
                    const int d0 = dt * 32 + 8 * jq + 4 * h;
                    float4 o;
                    o.x = oacc[dt][4 * jq + 0] * inv;
                    o.y = oacc[dt][4 * jq + 1] * inv;
                    o.z = oacc[dt][4 * jq + 2] * inv;
                    o.w = oacc[dt][4 * jq + 3] * inv;
                    *reinterpret_cast<float4*>(wo + d0) = o;
                }
            if (h == 0) p.ws_lse[prow] = lse2;
        }
    }
}

// Merge split partials: one packed row per 32 threads, 4 head-dim lanes per thread.  Rows of
// requests with one split were written by the attention kernel and are skipped.  The
// 32 threads of a row first spread its (at most 64) split log-sum-exps over their lanes, so
// the max and the weights take two loads per thread, then add the partial outputs eight
// splits at a time with the loads issued together.
static_assert(kMaxPrefillSplits <= 64 && kMaxDecodeSplits <= 64, "the merge holds two splits per lane");
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnParams p) {
    const Shape& s = p.s;
    const int64_t gid = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int64_t rows_all = (int64_t)s.B * s.Hkv * p.rows_total;
    if (gid >= rows_all) return;
    const int lane = threadIdx.x & 31;
    const int row = static_cast<int>(gid / p.rows_total);
    const int r = static_cast<int>(gid - (int64_t)row * p.rows_total);
    const int b = row / s.Hkv;
    const int hk = row - b * s.Hkv;
    const int nsplit = p.sp[b];
    if (nsplit == 1) return;  // the attention kernel wrote this request's rows directly
    if (p.ws_unsplit && *p.ws_unsplit) return;  // so it did for every row of an unsplit launch
    const int t = r / s.G;
    const int g = r - t * s.G;
    // lane holds splits lane and lane + 32
    const float ls0 = lane < nsplit ? p.ws_lse[(int64_t)lane * rows_all + gid] : -__builtin_inff();
    const float ls1 = lane + 32 < nsplit ? p.ws_lse[(int64_t)(lane + 32) * rows_all + gid] : -__builtin_inff();
    float mx = fmaxf(ls0, ls1);
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 32));
    const bool any = mx != -__builtin_inff();
    const float w0 = any ? __builtin_amdgcn_exp2f(ls0 - mx) : 0.0f;  // 0 for absent or empty splits
    const float w1 = any ? __builtin_amdgcn_exp2f(ls1 - mx) : 0.0f;
    float wsum = w0 + w1;
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) wsum += __shfl_xor(wsum, o, 32);
    float4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const float* wo = p.ws_o + gid * 128 + 4 * lane;
    for (int sp0 = 0; sp0 < nsplit; sp0 += 8) {
        float4 o[8];
        float wgt[8];
        // the partials' loads do not wait for the weights; a split with weight 0 (no keys)
        // is dropped by a select, so whatever its slot holds never reaches the sum
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int sp = sp0 + u;
            o[u] = sp < nsplit ? *reinterpret_cast<const float4*>(wo + (int64_t)sp * rows_all * 128)
                               : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int sp = sp0 + u;
            const float wa = __shfl(w0, sp & 31, 32);
            const float wb = __shfl(w1, sp & 31, 32);
            wgt[u] = sp < nsplit ? (sp < 32 ? wa : wb) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const bool use = wgt[u] != 0.0f;
            acc.x += use ? wgt[u] * o[u].x : 0.0f;
            acc.y += use ? wgt[u] * o[u].y : 0.0f;
            acc.z += use ? wgt[u] * o[u].z : 0.0f;
            acc.w += use ? wgt[u] * o[u].w : 0.0f;
        }
    }
    const float inv = wsum > 0.0f ? 1.0f / wsum : 0.0f;
    const int hq = hk * s.G + g;
    uint16_t* op = p.out.data + b * p.out.sb + (int64_t)t * p.out.st + (int64_t)hq * p.out.sh + 4 * lane;
    f32x4_t o4 = {acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
    *reinterpret_cast<bf16x4_t*>(op) = __builtin_convertvector(o4, bf16x4_t);
    if (p.lse && lane == 0)
        p.lse[((int64_t)b * s.Hq + hq) * s.Lq + t] =
            wsum > 0.0f ? (mx + __log2f(wsum)) * 0.69314718055994531f : -__builtin_inff();
}

// ---------------------------------------------------------------------------------------
// Dense decode with at most 16 packed query rows per KV row (q_len * G <= 16), e.g. one new
// token per request.  The work is HBM-bound (every cached byte is read once) and too narrow
// for 32-row tiles, so the shape differs from attn_fwd_kernel:
//  - 16x16x32 MFMAs (v_mfma_f32_16x16x32_bf16): S^T = K Q^T over 16-key tiles and
//    O^T += V^T P^T over 16-wide head-dim tiles, with the 16 packed rows as the N dimension;
//  - each of the 8 waves runs its own stream of blocks (e0 + w, e0 + w + 8, ...) with its
//    own online softmax, so eight blocks are in flight per CU and the waves' MFMA, softmax
//    and memory phases overlap; the eight partial results merge through LDS at the end;
//  - K goes straight from HBM into the MFMA A-operand registers (each lane loads 16 bytes
//    of one key row per 32-d step); V goes through the wave's own 16 KB of LDS (LDS DMA,
//    16-byte chunk c of row r at c ^ 2 (r & 7)) to be read transposed by ds_read_b64_tr_b16.
// The A-row -> key map of the P^T operand is permuted so that P comes straight out of the
// S^T accumulators: k-index (g, i) of 32-key step ks is key 32 ks + 16 (i / 4) + 4 g + i % 4
// for lane group g = lane / 16, and the transposed V reads follow the same map.
constexpr int kDecWaves = 8;
constexpr int kDecRows = 16;
constexpr int kDecVBytes = 64 * 256;
constexpr int kDecOStride = 132;  // floats per row of a wave's partial O in LDS (padded)

__global__ __launch_bounds__(kDecWaves * 64) void attn_decode_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[kDecWaves * kDecVBytes];

    const int L = blockIdx.x;
    const int x = L & 7;
    int k = L >> 3;
    const Shape& s = p.s;
    int row, b, split;
    if (p.use_rows) {
        int i = p.xoff[x];
        const int iend = p.xoff[x + 1];
        for (; i < iend; ++i) {
            const int items = p.xcnt[i];
            if (k < items) break;
            k -= items;
        }
        if (i >= iend) return;
        row = p.xrow[i];
        b = row / s.Hkv;
        split = p.xlo[i] + k;
    } else {
        const int W = x * p.per_xcd + k;
        if (W >= p.total_items) return;
        b = 0;
        while (b + 1 < s.B && p.ioff[b + 1] <= W) ++b;
        const int per_row = p.sp[b];
        row = b * s.Hkv + (W - p.ioff[b]) / per_row;
        split = (W - p.ioff[b]) % per_row;
    }
    const int hk = row - b * s.Hkv;
    const int nsplit = p.sp[b];
    const int G = s.G;
    const int R = p.rows_total;
    const int qpos0 = p.qpos0[b];
    const int nkb = p.nkb[b];  // the last query row sees every block
    const int chunk = (nkb + nsplit - 1) / nsplit;
    const int e0 = min(nkb, split * chunk);
    const int e1 = min(nkb, e0 + chunk);
    const int e_mask = (qpos0 + 1) >> 6;  // blocks from here on hold keys past query row 0

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l = tid & 63;
    const int n = l & 15;  // packed query row (N index)
    const int g = l >> 4;  // lane group (K index block)

    // Q^T (B operand of S^T): lane (n, g) holds Q[row n][32 j + 8 g .. + 7] for step j
    const bool qvalid = n < R;
    const int qt = qvalid ? n / G : 0;
    const int qg = qvalid ? n - qt * G : 0;
    bf16x8_t qf[4];
    {
        const uint16_t* qp = p.q.data + b * p.q.sb + (int64_t)qt * p.q.st + (int64_t)(hk * G + qg) * p.q.sh + 8 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (qvalid) {
                qf[j] = *reinterpret_cast<const bf16x8_t*>(qp + 32 * j);
            } else {
                u32x4_t z = {0u, 0u, 0u, 0u};
                qf[j] = __builtin_bit_cast(bf16x8_t, z);
            }
        }
    }
    const int qpos = qpos0 + qt;  // absolute position of this lane's query row

    const uint16_t* kbase_row = p.k.data + b * p.k.sb + hk * p.k.sh;
    const uint16_t* vbase_row = p.v.data + b * p.v.sb + hk * p.v.sh;
    const int32_t* kpt = p.k.page_table ? p.k.page_table + (int64_t)row * p.k.pts : nullptr;
    const int32_t* vpt = p.v.page_table ? p.v.page_table + (int64_t)row * p.v.pts : nullptr;
    const int kstok_b = static_cast<int>(p.k.stok) * 2;
    const int vstok_b = static_cast<int>(p.v.stok) * 2;
    const int kv_tokens = qpos0 + s.Lq;
    uint8_t* vbuf = smem + w * kDecVBytes;

    // A step is half a block (32 keys).  K (A operand of S^T) for key tile kt and 32-d step
    // j: lane (n, g) loads the 16 bytes at d = 32 j + 8 g of the half's key row 16 kt + n.
    // Buffer ranges end after the block's last existing token (rows past kv_len read as
    // zeros).
    int k_off[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) k_off[kt] = (16 * kt + n) * kstok_b + 16 * g;
    // V DMA: instruction i writes the half's LDS rows 4 i .. 4 i + 3; lane L fills row
    // 4 i + L / 16 at chunk position L & 15, which holds global chunk (L & 15) ^ 2 (row & 7).
    int v_goff[2];
#pragma unroll
    for (int par = 0; par < 2; ++par)
        v_goff[par] = (l >> 4) * vstok_b + (((l & 15) ^ (2 * (4 * par + (l >> 4)))) * 16);
    // V^T fragment (A operand of O^T) for d-tile dt: lane (a = l & 15, g) reads 8 bytes at
    // half row 16 hh + 4 g + a / 4, d = 16 dt + 4 (a & 3).
    int v_off[8];
    {
        const int a = l & 15;
        const int rr = 4 * g + (a >> 2);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) v_off[dt] = rr * 256 + 32 * (dt ^ (rr & 7)) + 8 * (a & 3);
    }

    // Two register sets for K and two 8 KB LDS halves for V: the loads of step st + 1 are in
    // flight while step st is computed.  One step is 8 K loads + 8 V DMA loads per wave.
    u32x4_t kf[2][2][4];
    uint8_t* vhalf[2] = {vbuf, vbuf + kDecVBytes / 2};
    auto block_rsrc = [&](const uint16_t* base, const int32_t* pt, int32_t max_page, int64_t sblk, int kb,
                          int stok_b) {
        const int64_t phys = pt ? clamp_page(sload(pt + kb), max_page) : kb;
        const int rows = min(kv_tokens - kb * 64, 64);
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base + phys * sblk), 0, rows * stok_b,
                                                 0x00020000);
    };
    const int nb_w = e0 + w < e1 ? (e1 - 1 - (e0 + w)) / kDecWaves + 1 : 0;  // this wave's blocks
    const int nsteps = 2 * nb_w;
    auto step_block = [&](int st) { return e0 + w + kDecWaves * (st >> 1); };
    auto issue = [&](int st, int set) {
        const int kb = step_block(st);
        const int half = st & 1;
        const __amdgpu_buffer_rsrc_t rk = block_rsrc(kbase_row, kpt, p.k.max_page, p.k.sblk, kb, kstok_b);
        const __amdgpu_buffer_rsrc_t rv = block_rsrc(vbase_row, vpt, p.v.max_page, p.v.sblk, kb, vstok_b);
        const int kh = 32 * half * kstok_b;
        const int vh = 32 * half * vstok_b;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
                kf[set][kt][j] = __builtin_amdgcn_raw_buffer_load_b128(rk, kh + k_off[kt] + 64 * j, 0, 0);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, to_lds(vhalf[set] + i * 1024), 16,
                                                     vh + v_goff[i & 1] + 4 * i * vstok_b, 0, 0, 0);
    };

    const float sl2 = p.scale_log2;
    f32x4_t oacc[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) oacc[dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -__builtin_inff();
    float l_run = 0.0f;
    const bf16x2_t ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};

    auto compute = [&](int st, int set) {
        const int kb = step_block(st);
        const int half = st & 1;
        f32x4_t sacc[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) sacc[kt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
                sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kf[set][kt][j]), qf[j],
                                                                  sacc[kt], 0, 0, 0);
        if (kb >= e_mask) {
            // value i of tile kt is key 64 kb + 32 half + 16 kt + 4 g + i
            const int vis = qpos - kb * 64 - 32 * half - 4 * g;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (16 * kt + i > vis) sacc[kt][i] = -__builtin_inff();
        }
        float mx = -__builtin_inff();
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sacc[kt][i]);
        mx = xor32_max(xor16_max(mx)) * sl2;
        float alpha = 1.0f;
        if (mx > m_run + kRescale) {
            alpha = __builtin_amdgcn_exp2f(m_run - mx);
            m_run = mx;
            l_run *= alpha;
        }
        if (__ballot(alpha != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) oacc[dt] *= alpha;
        }
        const float m_use = m_run == -__builtin_inff() ? 0.0f : m_run;
        f32x8_t pv8;
#pragma unroll
        for (int i = 0; i < 8; ++i) pv8[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[i >> 2][i & 3], sl2, -m_use));
        const bf16x8_t pf = __builtin_convertvector(pv8, bf16x8_t);
        // the normaliser sums the bf16-rounded weights the PV product uses
        l_run = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf, pf, 0, 1), ones, l_run, false);
        l_run = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf, pf, 2, 3), ones, l_run, false);
        l_run = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf, pf, 4, 5), ones, l_run, false);
        l_run = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf, pf, 6, 7), ones, l_run, false);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(to_lds_v4(vhalf[set] + v_off[dt]));
            const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(to_lds_v4(vhalf[set] + v_off[dt] + 4096));
            const bf16x8_t a = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pf, oacc[dt], 0, 0, 0);
        }
    };

    // nsteps is even: both halves of every block
    if (nsteps > 0) issue(0, 0);
    for (int st = 0; st < nsteps; st += 2) {
        issue(st + 1, 1);
        asm volatile("s_waitcnt vmcnt(16)" ::: "memory");  // step st has landed
        compute(st, 0);
        if (st + 2 < nsteps) {
            // the transposed reads of step st have returned before the DMA reuses its half
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(st + 2, 0);
            asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        } else {
            wait_dma();
        }
        compute(st + 1, 1);
    }

    // ---- merge the eight waves' partial results through LDS ----
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    __syncthreads();  // every wave is done with its V rows
    float* mo = reinterpret_cast<float*>(smem);
    float* ml = mo + kDecWaves * kDecRows * kDecOStride;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
        *reinterpret_cast<f32x4_t*>(mo + (w * kDecRows + n) * kDecOStride + 16 * dt + 4 * g) = oacc[dt];
    if (g == 0) {
        ml[(w * kDecRows + n) * 2 + 0] = m_run;
        ml[(w * kDecRows + n) * 2 + 1] = l_run;
    }
    __syncthreads();
    const int orow = tid >> 5;  // 16 rows x 32 threads, 4 head-dim values each
    const int d4 = (tid & 31) * 4;
    if (orow >= R) return;
    float mx = -__builtin_inff();
#pragma unroll
    for (int v = 0; v < kDecWaves; ++v) mx = fmaxf(mx, ml[(v * kDecRows + orow) * 2]);
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float wsum = 0.0f;
    if (mx != -__builtin_inff()) {
#pragma unroll
        for (int v = 0; v < kDecWaves; ++v) {
            const float wv = __builtin_amdgcn_exp2f(ml[(v * kDecRows + orow) * 2] - mx);
            wsum += wv * ml[(v * kDecRows + orow) * 2 + 1];
            acc += wv * *reinterpret_cast<const f32x4_t*>(mo + (v * kDecRows + orow) * kDecOStride + d4);
        }
    }
    const float inv = wsum > 0.0f ? 1.0f / wsum : 0.0f;
    const float lse2 = wsum > 0.0f ? mx + __log2f(wsum) : -__builtin_inff();
    acc *= inv;
    const int ot = orow / G;
    const int og = orow - ot * G;
    if (nsplit == 1) {
        const int hq = hk * G + og;
        uint16_t* op = p.out.data + b * p.out.sb + (int64_t)ot * p.out.st + (int64_t)hq * p.out.sh + d4;
        *reinterpret_cast<bf16x4_t*>(op) = __builtin_convertvector(acc, bf16x4_t);
        if (p.lse && (tid & 31) == 0) p.lse[((int64_t)b * s.Hq + hq) * s.Lq + ot] = lse2 * 0.69314718055994531f;
    } else {
        const int64_t prow = ((int64_t)split * (s.B * s.Hkv) + row) * R + orow;
        *reinterpret_cast<f32x4_t*>(p.ws_o + prow * 128 + d4) = acc;
        if ((tid & 31) == 0) p.ws_lse[prow] = lse2;
    }
}

}  // namespace

bool attn_uses_decode_kernel(const Shape& s, bool dense) {
    return dense && s.Lq * s.G <= kDecRows;
}

void attn_plan(const Shape& s, const int32_t* nkb, int forced, bool dense, SplitPlan* plan) {
    // One workgroup is resident per CU (128 KB of LDS).  Without a forced count, the
    // decode kernel splits each request's block list so its work items carry about the
    // same number of blocks as everyone else's (total work / slots); attn_fwd_kernel uses
    // one split count for all requests (below).  Both keep a minimum number of blocks per
    // split and at most the entry point's maximum of splits.
    //  - indexed prefill (attn_fwd_kernel): about one round of workgroups (256 slots) for
    //    requests of one length, two (512) for ragged batches, at least ~16 blocks per
    //    split, at most 16 splits;
    //  - dense decode with <= 16 rows (attn_decode_kernel): one round (256 slots), at least
    //    4 blocks per split, at most 32 splits.  Its eight waves stream blocks on their own,
    //    so one long item per CU beats two shorter ones (64 splits of a 128K-token cache,
    //    two rounds: 107.6 vs 99.6 us for 32), while a short cache gains from more CUs even
    //    when some waves of each item idle (32 Q / 8 KV heads: 4K tokens 26.3 -> 11.1 us,
    //    16K 30.3 -> 21.1 us, four 4K requests 30.0 -> 19.5 us against a floor of 32 blocks
    //    per split; 4 blocks per split at 1K tokens: 9.9 us, 9.0 and 9.5 us for 8 and 16 splits).
    //  - dense decode with more rows runs attn_fwd_kernel with the prefill sizing and up to
    //    64 splits.
    const bool dec = attn_uses_decode_kernel(s, dense);
    plan->may_unsplit = 0;
    const int slots = dec ? 256 : 512;
    const int min_blocks = dec ? 4 : 16;
    const int max_splits = dec ? 32 : dense ? kMaxDecodeSplits : kMaxPrefillSplits;
    const int rows_total = s.Lq * s.G;
    const int ntiles = dec ? 1 : (rows_total + kBM - 1) / kBM;
    double total = 0.0;
    int nkb_max = 1;
    for (int b = 0; b < s.B; ++b) {
        total += (double)s.Hkv * ntiles * nkb[b];
        nkb_max = max(nkb_max, nkb[b]);
    }
    const double item_blocks = total / slots;
    if (!dec && forced <= 0) {
        // attn_fwd_kernel: one split count for every request.  Splitting in proportion to
        // each request's blocks measured slower on ragged batches (config 4: 380 vs 319 us
        // sparse, 2386 vs 2077 us dense), and the blocks a request selects are device data
        // the host does not see.
        //  - Requests of one length: at most one round of work items (one per CU).  Their
        //    rows' lists have near-equal lengths, so the items stay balanced, and fewer
        //    splits write fewer partials for the merge (config 2, 128 row tiles: 2 splits
        //    513 us, 4 splits 522 us, 8 splits 549 us).  The count rounds down: a partial
        //    second round costs a whole item's time (28 Q / 4 KV heads, 16K tokens, chunk
        //    512, 56 row tiles: 5 splits, 280 items, 195 us against 134 us for 4).  Row
        //    tiles that fill three quarters of the CUs run unsplit (config-3 chunks, 256
        //    tiles: no partials or merge).
        //  - Ragged batches: about two rounds, which balances their long rows against the
        //    short ones.
        bool same_len = true;
        for (int b = 1; b < s.B; ++b) same_len = same_len && nkb[b] == nkb[0];
        const int units = s.B * s.Hkv * ntiles;
        forced = same_len ? 256 / units : static_cast<int>(slots / (double)units + 0.5);
        forced = min(forced, max(1, nkb_max / min_blocks));
        forced = max(1, min(forced, max_splits));
        if (same_len && units * 4 >= 3 * 256) forced = 1;
        // ragged batches with that many row tiles: the kernel decides from the selected
        // counts (even counts: one round of unsplit tiles; config 4 at 20 % keep 278-281 vs
        // 293-295 us split, while its dense tables need the split, 2.1 vs 3.2 ms)
        plan->may_unsplit = !same_len && units * 4 >= 3 * 256 && forced > 1;
    }
    plan->max = 1;
    plan->off[0] = 0;
    for (int b = 0; b < s.B; ++b) {
        const int nb = nkb[b];
        int sb = forced;
        if (forced <= 0) {
            sb = static_cast<int>(nb / item_blocks + 0.5);
            sb = min(sb, max(1, nb / min_blocks));
            sb = max(1, min(sb, max_splits));
        }
        plan->s[b] = sb;
        plan->max = max(plan->max, sb);
        plan->off[b + 1] = plan->off[b] + s.Hkv * ntiles * sb;
    }
    const int rows = s.B * s.Hkv;
    plan->use_rows = rows <= kPlanRows;
    if (!plan->use_rows) {
        plan->per_xcd = (plan->off[s.B] + 7) / 8;
        return;
    }
    // Placement units on the 8 XCDs.  A unit is a KV row and a range of its splits; the row
    // tiles of a unit stream the same blocks, so they share the XCD's L2, and different
    // split ranges of a row are disjoint parts of its block list (placing them apart
    // duplicates only the row's query reads).
    //  - Requests of one length over a multiple of 8 rows: whole rows, longest first, each
    //    to the least-loaded XCD (config 2 and 3: one or more rows per XCD).
    //  - Otherwise (rows that do not divide over the XCDs, or ragged lengths): single
    //    splits, dealt round-robin over the XCDs request by request, so every XCD gets an
    //    equal share of every request's work whatever the rows' selected counts turn out to
    //    be (the host only knows their past lengths); each XCD runs its units longest first.
    bool same_len = true;
    for (int b = 1; b < s.B; ++b) same_len = same_len && nkb[b] == nkb[0];
    int nunits = 0;
    for (int r = 0; r < rows; ++r) nunits += plan->s[r / s.Hkv];
    // (a launch that may run unsplit keeps whole rows: each XCD's tiles then fit one round)
    const bool split_units = (rows % 8 != 0 || !same_len) && nunits <= kPlanRows && !plan->may_unsplit;
    int unit_row[kPlanRows], unit_lo[kPlanRows], unit_cnt[kPlanRows];
    double unit_work[kPlanRows];  // blocks x row tiles the unit's items stream
    int units = 0;
    for (int r = 0; r < rows; ++r) {
        const int sp = plan->s[r / s.Hkv];
        const int m = split_units ? sp : 1;
        for (int g = 0; g < m; ++g) {
            const int lo = g * sp / m;
            const int hi = (g + 1) * sp / m;
            unit_row[units] = r;
            unit_lo[units] = lo;
            unit_cnt[units] = hi - lo;
            unit_work[units] = (double)nkb[r / s.Hkv] * ntiles * (hi - lo) / sp;
            ++units;
        }
    }
    int xcd_of[kPlanRows];
    double load[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int items[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (split_units) {
        for (int u = 0; u < units; ++u) xcd_of[u] = u % 8;  // request-major unit order
    } else {
        int order[kPlanRows];
        for (int u = 0; u < units; ++u) order[u] = u;
        for (int i = 1; i < units; ++i) {  // longest first, stable
            const int u = order[i];
            int j = i;
            while (j > 0 && unit_work[order[j - 1]] < unit_work[u]) {
                order[j] = order[j - 1];
                --j;
            }
            order[j] = u;
        }
        for (int i = 0; i < units; ++i) {
            const int u = order[i];
            int x = 0;
            for (int c = 1; c < 8; ++c)
                if (load[c] < load[x] || (load[c] == load[x] && items[c] < items[x])) x = c;
            xcd_of[u] = x;
            load[x] += unit_work[u];
            items[x] += ntiles * unit_cnt[u];
        }
    }
    // each XCD's units, longest first (stable)
    int nunit[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint16_t lists[8][kPlanRows];
    for (int x = 0; x < 8; ++x) items[x] = 0;
    for (int u = 0; u < units; ++u) {
        const int x = xcd_of[u];
        int j = nunit[x]++;
        while (j > 0 && unit_work[lists[x][j - 1]] < unit_work[u]) {
            lists[x][j] = lists[x][j - 1];
            --j;
        }
        lists[x][j] = static_cast<uint16_t>(u);
        items[x] += ntiles * unit_cnt[u];
    }
    plan->xoff[0] = 0;
    plan->per_xcd = 0;
    for (int x = 0; x < 8; ++x) {
        for (int i = 0; i < nunit[x]; ++i) {
            const int u = lists[x][i];
            plan->xrow[plan->xoff[x] + i] = static_cast<uint16_t>(unit_row[u]);
            plan->xlo[plan->xoff[x] + i] = static_cast<uint8_t>(unit_lo[u]);
            plan->xcnt[plan->xoff[x] + i] = static_cast<uint8_t>(unit_cnt[u]);
        }
        plan->xoff[x + 1] = plan->xoff[x] + nunit[x];
        plan->per_xcd = max(plan->per_xcd, items[x]);
    }
}

void attn_positions(const Shape& s, const PastBlocks& pb, const int32_t* kv_len, int32_t* qpos0, int32_t* nkb) {
    for (int b = 0; b < s.B; ++b) {
        if (kv_len) {  // decode: the q_len query rows are the last positions of kv_len
            qpos0[b] = kv_len[b] - s.Lq;
            nkb[b] = (kv_len[b] + 63) / 64;
        } else {       // chunked prefill: the chunk starts at block P_b
            qpos0[b] = 64 * pb.p[b];
            nkb[b] = pb.p[b] + s.Qb;
        }
    }
}

int attn_pick_splits(const Shape& s, const PastBlocks& pb, const int32_t* kv_len) {
    int32_t qpos0[CA_MAX_BATCH], nkb[CA_MAX_BATCH];
    attn_positions(s, pb, kv_len, qpos0, nkb);
    SplitPlan plan;
    attn_plan(s, nkb, 0, kv_len != nullptr, &plan);
    return plan.max;
}

int64_t attn_workspace_bytes(const Shape& s, int num_splits) {
    if (num_splits <= 1) return 0;
    const int64_t rows_all = (int64_t)s.B * s.Hkv * s.Lq * s.G;
    // partials (128 values + log2-LSE per split and packed row), then the unsplit flag
    return (int64_t)num_splits * rows_all * (128 + 1) * (int64_t)sizeof(float) + 16;
}

hipError_t launch_attn(const AttnArgs& a, hipStream_t stream) {
    AttnParams p;
    p.s = a.s;
    p.q = a.q;
    p.k = a.k;
    p.v = a.v;
    p.table = a.table;
    p.table_stride = a.table_stride;
    p.counts = a.counts;
    p.pb = a.pb;
    p.scale_log2 = a.scale * 1.4426950408889634f;
    p.out = a.out;
    p.lse = a.lse;
    p.rows_total = a.s.Lq * a.s.G;
    p.ntiles = (p.rows_total + kBM - 1) / kBM;
    int32_t nkb[CA_MAX_BATCH];
    attn_positions(a.s, a.pb, a.kv_len, p.qpos0, nkb);
    for (int b = 0; b < CA_MAX_BATCH; ++b) p.nkb[b] = b < a.s.B ? nkb[b] : 0;
    for (int b = a.s.B; b < CA_MAX_BATCH; ++b) p.qpos0[b] = 0;
    SplitPlan plan;
    attn_plan(a.s, nkb, a.num_splits, a.kv_len != nullptr, &plan);
    for (int b = 0; b < CA_MAX_BATCH; ++b) p.sp[b] = b < a.s.B ? plan.s[b] : 1;
    for (int b = 0; b <= CA_MAX_BATCH; ++b) p.ioff[b] = b <= a.s.B ? plan.off[b] : plan.off[a.s.B];
    p.total_items = plan.off[a.s.B];
    p.per_xcd = plan.per_xcd;
    p.use_rows = plan.use_rows;
    for (int x = 0; x < 9; ++x) p.xoff[x] = plan.use_rows ? plan.xoff[x] : 0;
    for (int i = 0; i < kPlanRows; ++i) {
        const bool used = plan.use_rows && i < plan.xoff[8];
        p.xrow[i] = used ? plan.xrow[i] : 0;
        p.xlo[i] = used ? plan.xlo[i] : 0;
        p.xcnt[i] = used ? plan.xcnt[i] : 1;
    }
    const int64_t rows_all = (int64_t)a.s.B * a.s.Hkv * p.rows_total;
    p.ws_o = plan.max > 1 ? static_cast<float*>(a.workspace) : nullptr;
    p.ws_lse = plan.max > 1 ? p.ws_o + (int64_t)plan.max * rows_all * 128 : nullptr;
    p.ws_unsplit = plan.max > 1 && plan.may_unsplit && a.table
                       ? reinterpret_cast<int32_t*>(p.ws_lse + (int64_t)plan.max * rows_all)
                       : nullptr;
    {
        int max_tokens = 0;
        for (int b = 0; b < a.s.B; ++b) max_tokens = max(max_tokens, p.qpos0[b] + a.s.Lq);
        const int64_t stok = max(a.k.stok, a.v.stok);
        p.row_res = a.k.page_table == nullptr && a.v.page_table == nullptr && a.k.sblk == 64 * a.k.stok &&
                    a.v.sblk == 64 * a.v.stok && (int64_t)max_tokens * stok * 2 + 64 * stok * 2 < (int64_t{1} << 31);
    }
    if (a.table)
        hipLaunchKernelGGL((attn_fwd_kernel<kNW, true>), dim3(p.per_xcd * 8), dim3(kNW * 64), 0, stream, p);
    else if (attn_uses_decode_kernel(a.s, true))
        hipLaunchKernelGGL(attn_decode_kernel, dim3(p.per_xcd * 8), dim3(kDecWaves * 64), 0, stream, p);
    else
        hipLaunchKernelGGL((attn_fwd_kernel<kNW, false>), dim3(p.per_xcd * 8), dim3(kNW * 64), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || plan.max <= 1) return e;
    const int64_t blocks = (rows_all + 7) / 8;
    hipLaunchKernelGGL(attn_merge_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace ca
