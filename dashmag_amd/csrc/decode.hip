// Attention decode against a key-value cache (crates/dash-ops/src/attention.rs:732,
// attention/cube.rs:1126-1214, kernels.rs:2052-2239): flash-decoding. Pass 1 splits each
// sequence's keys into fixed-size spans; one workgroup reads a span of K and V rows once for
// all the query heads of a key-value head's group (the GQA reuse), and writes a normalised
// partial output and its log-sum-exp in f32. Pass 2 merges the spans by their log-sum-exp.
//
// Bandwidth-bound. The split pass runs its products on MFMA (decode_split_mfma) at D = 64, 128
// and 256 for bf16/f16: a GQA group's query heads read the same key rows, so the scores of a block
// of keys are one small product, cheaper on the matrix units than as per-head dot products on the
// vector units. f32 and other shapes take decode_generic.
#include <mutex>
#include <string>

#include "attention_kernels.h"
#include "dm_common.h"
#include "mfma.h"

namespace dm {

constexpr int kDecodeMinSpan = 128;          // fewest keys a workgroup takes (one block a wavefront)
constexpr int kDecodeWorkgroupsMfma = 4096;  // the split count aims at about this many workgroups

// Where the cache keeps sequence b's keys. Dense: rows b * S .. b * S + S - 1 of k, v
// [B, S, Hkv, D]. Packed: rows offsets[b] .. offsets[b + 1] - 1 of k, v [N, Hkv, D]
// (offsets = cu_seqlens_k, [B + 1] int32), at most S of them. Paged: key j of sequence b is row
// j % page_size of page block_table[b * max_pages + j / page_size] of k, v
// [num_pages, page_size, Hkv, D]; a page index outside [0, num_pages) reads as zeros.
//
// Element strides: the query's along (batch, head); the cache's along (batch row or page, key,
// head), the key's t stride also the distance between a packed cache's rows.
struct KvMap {
    const int32_t *offsets;
    const int32_t *block_table;
    int64_t page_size, max_pages, num_pages;
    int64_t qb, qh;
    int64_t kb, kt, kh, vb, vt, vh;
};

// Sequence b's first cache row (dense and packed) and the number of keys it holds: lengths[b]
// (every key of its span without lengths), clamped to [0, its span].
__device__ __forceinline__ void kv_extent(const KvMap &m, int64_t b, int64_t S,
                                          const int32_t *lengths, int64_t &row0, int64_t &len) {
    int64_t cap = S;
    row0 = b * S;
    if (m.offsets) {
        row0 = m.offsets[b];
        const int64_t n = (int64_t)m.offsets[b + 1] - row0;
        cap = n < S ? n : S;
        if (cap < 0) cap = 0;
    }
    len = lengths ? (int64_t)lengths[b] : cap;
    if (len > cap) len = cap;
    if (len < 0) len = 0;
}

// Element offsets of sequence b's key 0 in the key and value caches (dense and packed), for
// row0 from kv_extent.
__device__ __forceinline__ int64_t kv_base_k(const KvMap &m, int64_t b, int64_t row0) {
    return m.offsets ? row0 * m.kt : b * m.kb;
}
__device__ __forceinline__ int64_t kv_base_v(const KvMap &m, int64_t b, int64_t row0) {
    return m.offsets ? row0 * m.vt : b * m.vb;
}

// Paged caches: the page holding key j of sequence b, or -1 when its index is out of range.
__device__ __forceinline__ int64_t kv_page(const KvMap &m, int64_t b, int64_t j) {
    const int64_t pg = m.block_table[b * m.max_pages + j / m.page_size];
    return pg >= 0 && pg < m.num_pages ? pg : -1;
}

// The splits of one (sequence, query head) merged by their log-sum-exp, by the 256 threads of a
// workgroup. The row's log-sum-exps go to LDS once (one load a thread) and become the splits'
// weights; then thread t sums, for the 4 columns of its 16-byte piece d4 = t % (D / 4), the
// splits s = t / (D / 4) + k * (1024 / D), four loads in flight at a time, and the split groups'
// sums are added in a fixed order through LDS. (A thread walking every split of its columns one
// dependent load after another took 6-8 us for a handful of rows.)
struct MergeLds {
    float w[4096];      // the splits' weights (nsplit <= 4096, span_of)
    float4 red[256];    // the split groups' partial sums
};
template <int DT>
__device__ __forceinline__ void merge_row(int64_t row, int64_t D, int nsplit,
                                          const float *__restrict__ part_o,
                                          const float *__restrict__ part_lse,
                                          void *__restrict__ o, MergeLds &ml) {
    float *wsm = ml.w;
    float4 *red = ml.red;
    const int tid = threadIdx.x;
    const float *pl = part_lse + row * nsplit;
    float mx = -INFINITY;
    for (int sp = tid; sp < nsplit; sp += 256) {
        const float x = pl[sp];
        wsm[sp] = x;
        mx = fmaxf(mx, x);
    }
    mx = wave_max(mx);
    __syncthreads();
    if ((tid & 63) == 0) red[tid >> 6].x = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0].x, red[1].x), fmaxf(red[2].x, red[3].x));
    float lsum = 0.f;
    for (int sp = tid; sp < nsplit; sp += 256) {
        const float w = M == -INFINITY ? 0.f : __expf(wsm[sp] - M);
        wsm[sp] = w;
        lsum += w;
    }
    lsum = wave_sum(lsum);
    __syncthreads();
    if ((tid & 63) == 0) red[tid >> 6].y = lsum;
    __syncthreads();
    const float L = (red[0].y + red[1].y) + (red[2].y + red[3].y);
    __syncthreads();
    const int nd4 = (int)(D / 4), groups = 256 / nd4;
    const int d4 = tid % nd4, grp = tid / nd4;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (grp < groups) {
        const float4 *po = (const float4 *)(part_o + row * nsplit * D) + d4;
        int sp = grp;
        for (; sp + 3 * groups < nsplit; sp += 4 * groups) {
            float4 x[4];
#pragma unroll
            for (int u = 0; u < 4; u++) x[u] = po[(int64_t)(sp + u * groups) * nd4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float w = wsm[sp + u * groups];
                acc.x += w * x[u].x, acc.y += w * x[u].y, acc.z += w * x[u].z, acc.w += w * x[u].w;
            }
        }
        for (; sp < nsplit; sp += groups) {
            const float4 x = po[(int64_t)sp * nd4];
            const float w = wsm[sp];
            acc.x += w * x.x, acc.y += w * x.y, acc.z += w * x.z, acc.w += w * x.w;
        }
    }
    red[tid] = acc;
    __syncthreads();
    if (tid < nd4) {
        float4 a = red[tid];
        for (int g = 1; g < groups; g++) {
            const float4 b = red[g * nd4 + tid];
            a.x += b.x, a.y += b.y, a.z += b.z, a.w += b.w;
        }
        const float inv = L > 0.f ? 1.f / L : 0.f;
        const int64_t ob = row * D + tid * 4;
        st<DT>(o, ob, a.x * inv);
        st<DT>(o, ob + 1, a.y * inv);
        st<DT>(o, ob + 2, a.z * inv);
        st<DT>(o, ob + 3, a.w * inv);
    }
    __syncthreads();
}

// The split pass on MFMA (D = 64, 128 or 256). Each wavefront sweeps its quarter of the split in
// blocks of 32 keys: the block's K and V rows arrive by coalesced 16-byte loads (64 / (D / 8) rows
// per load), go to the wavefront's own LDS tiles, and the next block's loads are in flight while this block is
// used. Per block, S^T = K q^T (32 keys x the group's heads, padded to 32 columns) and
// O^T += V^T P^T (4 tiles of 32 columns x the heads) run as 32x32x16 products: the scores'
// output layout (lane = head, rows = keys) is the B operand of the second product as it stands,
// and V^T comes from transposed LDS reads. Each lane keeps the online softmax of its head in f32.
//
// PAGED: the blocks start at keys that are multiples of 16, so each 16-key half of a block lies
// in one page (page_size is a multiple of 16). Per half, one wavefront-uniform read of the block
// table gives the page, and the half's buffer resource starts at the half's first visible key
// and spans only its visible keys: keys before the wavefront's range (negative offsets wrap past
// the end), past it, or on a page index out of range read as zeros, and their scores are -inf.
// At D = 256 a wavefront's staged block (64 registers per tensor), the queries' fragments and
// O^T need one wavefront per SIMD.
template <int DT, int G, bool PAGED, int D>
__global__ __launch_bounds__(256, D == 256 ? 1 : 2) void decode_split_mfma(
    int64_t S, int64_t Hq, int64_t Hkv, int64_t left, float scale, int nsplit, int span,
    const void *__restrict__ q, const void *__restrict__ k, const void *__restrict__ v,
    const int32_t *__restrict__ lengths, KvMap map, float *__restrict__ part_o,
    float *__restrict__ part_lse, void *__restrict__ out) {
    constexpr int NW = 4, BK = 32;
    constexpr int KS = D + 8, VS = D + 32;  // row strides (elements) of the row and transposed reads
    constexpr int LPR = D / 8, RPL = 64 / LPR, NLD = BK / RPL;  // lanes per row, rows per load, loads
    constexpr int KST = D / 16, DTN = D / 32;  // k-steps of the scores, 32-column tiles of O^T
    struct Tiles {
        uint16_t k[BK * KS];
        uint16_t v[BK * VS];
    };
    static_assert(sizeof(float) * NW * (G * D + 2 * G) <= sizeof(Tiles) * NW, "combine in tiles");
    __shared__ __align__(16) Tiles tiles[NW];
    const int kh = blockIdx.x, split = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 31, half = lane >> 5;

    int64_t row0, len;
    kv_extent(map, b, S, lengths, row0, len);
    int64_t lo = left >= 0 ? len - 1 - left : 0;
    if (lo < 0) lo = 0;
    const int64_t start = lo + (int64_t)split * span;
    int64_t end = start + span;
    if (end > len) end = len;

    // the queries as B operands: column = head col (zero past the group), k slots
    // d = 16 st + 4 h + e and 16 st + 8 + 4 h + e (the order of the key rows' A fragments)
    Frag8 qf[KST];
#pragma unroll
    for (int st = 0; st < KST; st++) {
        if (col < G) {
            const uint16_t *qp = (const uint16_t *)q + b * map.qb + (kh * G + col) * map.qh +
                                 st * 16 + half * 4;
            const uint2 a = *(const uint2 *)qp, c = *(const uint2 *)(qp + 8);
            qf[st].u = make_uint4(a.x, a.y, c.x, c.y);
        } else {
            qf[st].u = make_uint4(0, 0, 0, 0);
        }
    }
    const float qscale = scale * 1.4426950408889634f;

    const int64_t row_stride = map.kt * 2;  // bytes between consecutive keys (and values)
    const char *kb = (const char *)k + ((PAGED ? 0 : kv_base_k(map, b, row0)) + kh * map.kh) * 2;
    const char *vb = (const char *)v + ((PAGED ? 0 : kv_base_v(map, b, row0)) + kh * map.vh) * 2;
    // each wavefront sweeps a contiguous quarter of the split
    const int64_t per_wave = span / NW;
    const int64_t w0 = start + wave * per_wave;
    const int64_t w1 = min(w0 + per_wave, end);
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(kb + w0 * row_stride, 0xffffffffu);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vb + w0 * row_stride, 0xffffffffu);
    Tiles &t = tiles[wave];
    // one register set: a block's loads are issued as soon as the previous block is staged, and
    // are in flight while that block's products run
    struct Stage {
        uint4 k[NLD], v[NLD];
    };
    Stage sts;
    // PAGED: the pages of a block's two 16-key halves (-1: no visible key, or an index out of
    // range), looked up one block ahead of the block's loads
    struct Pages {
        int64_t pg[2];
    };
    auto pages_of = [&](int64_t j0) __attribute__((always_inline)) {
        Pages p;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int64_t h0 = j0 + 16 * h;
            const int64_t first = max(h0, w0), last = min(h0 + 16, w1);
            p.pg[h] = PAGED && first < last ? kv_page(map, b, first) : -1;
        }
        return p;
    };
    // block rows past the wavefront's range load row w1 - 1 again (their scores are -inf)
    auto load = [&](Stage &x, int64_t j0, const Pages &pages) __attribute__((always_inline)) {
        if constexpr (PAGED) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int64_t h0 = j0 + 16 * h;
                const int64_t first = max(h0, w0), last = min(h0 + 16, w1);
                const int64_t pg = pages.pg[h];
                const uint32_t bytes = pg >= 0 ? (uint32_t)((last - first) * row_stride) : 0u;
                // the half's first visible key within its page
                const int64_t kofs = pg >= 0 ? (pg * map.kb + first % map.page_size * map.kt) * 2 : 0;
                const int64_t vofs = pg >= 0 ? (pg * map.vb + first % map.page_size * map.vt) * 2 : 0;
                const __amdgpu_buffer_rsrc_t kh_rs = make_rsrc(kb + kofs, bytes);
                const __amdgpu_buffer_rsrc_t vh_rs = make_rsrc(vb + vofs, bytes);
                // the offset of key j0 + RPL u + lane / LPR from the half's first visible key: a
                // lane part and a wavefront-uniform part per load (negative before that key: it
                // wraps past the resource's range and reads zeros)
                const uint32_t lane_off = (uint32_t)((lane / LPR) * row_stride) + (lane % LPR) * 16;
                const int32_t ubase = __builtin_amdgcn_readfirstlane((int32_t)((j0 - first) * row_stride));
#pragma unroll
                for (int u = h * NLD / 2; u < (h + 1) * NLD / 2; u++) {
                    const uint32_t off = lane_off + (uint32_t)(ubase + (int32_t)(RPL * u * row_stride));
                    x.k[u] = buf_load16_nt(kh_rs, off);
                    x.v[u] = buf_load16_nt(vh_rs, off);
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < NLD; u++) {
                const int64_t key = min(j0 + RPL * u + lane / LPR, w1 - 1);
                const uint32_t off = (uint32_t)((key - w0) * row_stride) + (lane % LPR) * 16;
                x.k[u] = buf_load16_nt(krs, off);
                x.v[u] = buf_load16_nt(vrs, off);
            }
        }
    };
    auto stage = [&](const Stage &x) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NLD; u++) {
            const int r = RPL * u + lane / LPR, c = (lane % LPR) * 8;
            *(uint4 *)(t.k + r * KS + c) = x.k[u];
            *(uint4 *)(t.v + r * VS + c) = x.v[u];
        }
    };
    float m = -INFINITY, l = 0.f;
    f32x16_t acc[DTN];
#pragma unroll
    for (int dt = 0; dt < DTN; dt++) acc[dt] = zero16();
    auto block = [&](int64_t j0) __attribute__((always_inline)) {
        f32x16_t sc = zero16();
#pragma unroll
        for (int st = 0; st < KST; st++) sc = mfma32<DT>(row_frag(t.k, KS, 0, st * 16, lane), qf[st], sc);
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int64_t key = j0 + crow(i, lane);
            sc[i] = key < w1 && (!PAGED || key >= w0) ? sc[i] * qscale : -INFINITY;
            mx = fmaxf(mx, sc[i]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        // lazy rescale: the reference m moves (and O^T, l are rescaled) only when a head's
        // maximum grows past it by more than 2^8 (exponentials stay below 256); from -inf any
        // visible key moves it, and with nothing visible yet (m = -inf) every factor is 0
        const bool grow = mx > m + 8.f;
        if (__any(grow)) {
            const float mn = grow ? mx : m;
            const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mn);
            m = mn;
            l *= alpha;
#pragma unroll
            for (int dt = 0; dt < DTN; dt++)
#pragma unroll
                for (int i = 0; i < 16; i++) acc[dt][i] *= alpha;
        }
        const float ref = m == -INFINITY ? 0.f : m;
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            sc[i] = __builtin_amdgcn_exp2f(sc[i] - ref);
            ps += sc[i];
        }
        l += ps;
        const Frag8 p0 = c_frag<DT>(sc, 0), p1 = c_frag<DT>(sc, 1);
#pragma unroll
        for (int dt = 0; dt < DTN; dt++) {
            acc[dt] = mfma32<DT>(lds_tr_frag(t.v, VS, 0, dt * 32, lane), p0, acc[dt]);
            acc[dt] = mfma32<DT>(lds_tr_frag(t.v, VS, 16, dt * 32, lane), p1, acc[dt]);
        }
    };
    // (the loop is a single block: with the last block peeled off, as a separate copy after the
    // loop, the kernel measured 15% slower)
    // (a counted loop: with the exit test as a break the compiler kept O^T in vector registers
    // across it at D = 256 and spilled)
    if (w0 < w1) {
        const int64_t a0 = PAGED ? (w0 & ~(int64_t)15) : w0;
        const int nblk = (int)((w1 - a0 + BK - 1) / BK);
        Pages pn = pages_of(a0);
        load(sts, a0, pn);
        pn = pages_of(a0 + BK);
        for (int n = 0; n < nblk; n++) {
            const int64_t j0 = a0 + (int64_t)n * BK;
            stage(sts);
            load(sts, j0 + BK, pn);
            pn = pages_of(j0 + 2 * BK);
            block(j0);
        }
    }
    l += __shfl_xor(l, 32, 64);

    // the wavefronts' partial results through LDS (the tiles' space): [NW][G] m and l,
    // [NW][G][D] acc
    __syncthreads();
    float *sm_acc = (float *)tiles, *sm_m = sm_acc + NW * G * D, *sm_l = sm_m + NW * G;
    if (col < G) {
#pragma unroll
        for (int dt = 0; dt < DTN; dt++)
#pragma unroll
            for (int i = 0; i < 16; i++) sm_acc[(wave * G + col) * D + dt * 32 + crow(i, lane)] = acc[dt][i];
        if (half == 0) {
            sm_m[wave * G + col] = m;
            sm_l[wave * G + col] = l;
        }
    }
    __syncthreads();
    for (int x = threadIdx.x; x < G * D; x += 256) {
        const int g = x / D, d = x % D;
        float M = -INFINITY;
        for (int w = 0; w < NW; w++) M = fmaxf(M, sm_m[w * G + g]);
        float L = 0.f, A = 0.f;
        if (M != -INFINITY) {
            for (int w = 0; w < NW; w++) {
                const float f = __builtin_amdgcn_exp2f(sm_m[w * G + g] - M);
                L += sm_l[w * G + g] * f;
                A += sm_acc[(w * G + g) * D + d] * f;
            }
        }
        const int64_t pr = (b * Hq + kh * G + g) * nsplit + split;
        if (nsplit == 1) {
            // one split: its normalised partial is the output
            st<DT>(out, (b * Hq + kh * G + g) * D + d, L > 0.f ? A / L : 0.f);
            continue;
        }
        part_o[pr * D + d] = L > 0.f ? A / L : 0.f;
        if (d == 0) part_lse[pr] = L > 0.f ? (M + log2f(L)) * 0.6931471805599453f : -INFINITY;
    }
}

// Pass 2: merges the splits of one (sequence, query head) by their log-sum-exp, one workgroup a
// row. (Merging in the split kernel instead, by the last of a key-value head's splits to finish,
// measured slower: with release/acquire fences every workgroup wrote back and invalidated its
// L2, 5x the split pass's time; with write-through partial stores and a relaxed counter each
// workgroup waited on its stores' acknowledgement, 237 against 215 us on config 3.)
template <int DT>
__global__ __launch_bounds__(256) void decode_merge(int64_t rows, int64_t D, int nsplit,
                                                    const float *__restrict__ part_o,
                                                    const float *__restrict__ part_lse,
                                                    void *__restrict__ o) {
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    __shared__ MergeLds ml;
    merge_row<DT>(row, D, nsplit, part_o, part_lse, o, ml);
}

// The generic decode: the generic attention forward's arithmetic, one wavefront per
// (sequence, query head), for head widths, groups and dtypes the split kernels do not take, and
// for paged caches whose pages are not a multiple of 16 keys (a key on a page index out of range
// counts as zeros).
template <int DT, int NPL, bool PAGED>
__global__ __launch_bounds__(256) void decode_generic(int64_t B, int64_t S, int64_t Hq,
                                                      int64_t Hkv, int64_t D, int64_t left,
                                                      float scale, const void *q, const void *k,
                                                      const void *v, const int32_t *lengths,
                                                      KvMap map, void *o) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= B * Hq) return;
    const int64_t b = row / Hq, h = row % Hq, kh = h / (Hq / Hkv);
    int64_t row0, len;
    kv_extent(map, b, S, lengths, row0, len);
    int64_t lo = left >= 0 ? len - 1 - left : 0;
    if (lo < 0) lo = 0;
    float qr[NPL], acc[NPL];
    const int64_t qo = b * map.qb + h * map.qh;
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        int64_t d = lane + 64 * e;
        qr[e] = d < D ? ld<DT>(q, qo + d) : 0.f;
        acc[e] = 0.f;
    }
    const int64_t kseq = kv_base_k(map, b, row0) + kh * map.kh;
    const int64_t vseq = kv_base_v(map, b, row0) + kh * map.vh;
    float mx = -INFINITY, l = 0.f;
    for (int64_t j = lo; j < len; j++) {
        int64_t kr, vr;
        bool cr = true;  // false: a page index out of range (the key counts as zeros)
        if constexpr (PAGED) {
            const int64_t pg = kv_page(map, b, j), r = j % map.page_size;
            cr = pg >= 0;
            kr = pg * map.kb + r * map.kt + kh * map.kh;
            vr = pg * map.vb + r * map.vt + kh * map.vh;
        } else {
            kr = kseq + j * map.kt;
            vr = vseq + j * map.vt;
        }
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < NPL; e++) {
            int64_t d = lane + 64 * e;
            if (d < D && cr) s += qr[e] * ld<DT>(k, kr + d);
        }
        s = wave_sum(s) * scale;
        const float mn = fmaxf(mx, s);
        const float alpha = expf(mx - mn), p = expf(s - mn);
        l = l * alpha + p;
#pragma unroll
        for (int e = 0; e < NPL; e++) {
            int64_t d = lane + 64 * e;
            acc[e] = acc[e] * alpha + p * (d < D && cr ? ld<DT>(v, vr + d) : 0.f);
        }
        mx = mn;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        int64_t d = lane + 64 * e;
        if (d < D) st<DT>(o, row * D + d, acc[e] * inv);
    }
}

// The call's strides (elements): the descriptor's, or the contiguous layouts' (q [B, Hq, D];
// a dense cache [B, S, Hkv, D], a packed one [N, Hkv, D], pages [P, page_size, Hkv, D]).
static KvMap kv_strides(const dm_attention_desc *d, int64_t page_size) {
    KvMap m{};
    if (d->strided) {
        m.qb = d->sq.b, m.qh = d->sq.h;
        m.kb = d->sk.b, m.kt = d->sk.t, m.kh = d->sk.h;
        m.vb = d->sv.b, m.vt = d->sv.t, m.vh = d->sv.h;
    } else {
        const int64_t row = d->hkv * d->d, rows = page_size > 0 ? page_size : d->tk;
        m.qb = d->hq * d->d, m.qh = d->d;
        m.kb = m.vb = rows * row, m.kt = m.vt = row, m.kh = m.vh = d->d;
    }
    return m;
}

// The split kernels read keys and values with one row stride of at least a row, in 16-byte
// pieces; their shapes as below.
static bool split_takes(const dm_attention_desc *d, int64_t page_size = 0) {
    const int64_t g = d->hq / d->hkv;
    const KvMap m = kv_strides(d, page_size);
    const bool rows = m.kt == m.vt && m.kt >= d->d && m.qh % 8 == 0 && m.qb % 8 == 0 &&
                      m.kb % 8 == 0 && m.kt % 8 == 0 && m.kh % 8 == 0 && m.vb % 8 == 0 &&
                      m.vh % 8 == 0;
    return (d->dtype == DM_BF16 || d->dtype == DM_F16) &&
           (d->d == 64 || d->d == 128 || d->d == 256) && (g == 1 || g == 2 || g == 4 || g == 8) &&
           rows;
}

// A paged cache runs the split pass on MFMA for pages of a multiple of 16 keys; other page sizes
// take the generic kernel.
static bool paged_split_takes(const dm_attention_desc *d, int64_t page_size) {
    return split_takes(d, page_size) && page_size % 16 == 0;
}

static int64_t left_of(const dm_attention_desc *d) {
    const uint64_t span = (uint64_t)d->tk + 1;  // `bound(left, s + 1)`, reference.rs:449
    const uint64_t left = d->options.has_window ? d->options.window_left : DM_UNBOUNDED;
    return left < span ? (int64_t)left : -1;
}

// The most keys a sequence's query sees: the cache, or the window's left + 1 (the splits cover
// the visible keys only; they start at the window's first key).
static int64_t visible_of(const dm_attention_desc *d) {
    const int64_t left = left_of(d);
    return left >= 0 && left + 1 < d->tk ? left + 1 : d->tk;
}

static int span_of(const dm_attention_desc *d) {
    int64_t span = kDecodeMinSpan;
    const int64_t heads = d->b * d->hkv, keys = visible_of(d);
    // (at D = 256 one workgroup fills a compute unit, and its wavefronts' sweeps need length:
    // about one workgroup per compute unit measured best)
    const int64_t target = d->d == 256 ? kDecodeWorkgroupsMfma / 16 : kDecodeWorkgroupsMfma;
    while (span < keys && heads * ((keys + span - 1) / span) > target) span *= 2;
    return (int)span;
}

static int nsplit_of(const dm_attention_desc *d) {
    const int64_t span = span_of(d), keys = visible_of(d);
    return (int)((keys + span - 1) / span);
}

// The checks both entry points share; returns DM_OK or the refusal.
static int check_decode(const char *op, const dm_attention_desc *d) {
    const std::string o(op);
    if (!d) return refuse(o + ": null descriptor");
    if (d->b < 0 || d->tk < 0 || d->hq < 0 || d->hkv <= 0 || d->d < 0)
        return refuse(o + ": bad dimensions");
    if (d->hq % d->hkv != 0)
        return refuse(o + ": the query heads (" + std::to_string(d->hq) +
                      ") must be a multiple of the key-value heads (" + std::to_string(d->hkv) +
                      ")");
    if (d->dtype != DM_F32 && d->dtype != DM_BF16 && d->dtype != DM_F16)
        return refuse(o + ": dtype must be f32, bf16 or f16");
    if (d->d > 256) return refuse(o + ": head dimension above 256 is not implemented");
    if (d->strided && (d->sq.b < 0 || d->sq.h < 0 || !strides_ok(Strd{d->sk.b, d->sk.t, d->sk.h}) ||
                       !strides_ok(Strd{d->sv.b, d->sv.t, d->sv.h})))
        return refuse(o + ": strides must not be negative");
    return DM_OK;
}

// Launches the generic kernel, or the split pass and the merge.
static int run_decode(const char *op, const dm_attention_desc *d, bool split, bool paged,
                      const void *q, const void *k, const void *v, const int32_t *lengths,
                      const KvMap &map, void *o, void *workspace, hipStream_t st) {
    const std::string opn(op);
    const int64_t rows = d->b * d->hq;
    const float scale = scale_of(d);
    const int64_t left = left_of(d);
    if (!split) {
        const int npl = d->d <= 64 ? 1 : (d->d <= 128 ? 2 : 4);
        dim3 grid((unsigned)((rows + 3) / 4));
#define DEC_GEN2(DT, NPL, PG)                                                               \
    decode_generic<DT, NPL, PG><<<grid, 256, 0, st>>>(d->b, d->tk, d->hq, d->hkv, d->d, left, \
                                                      scale, q, k, v, lengths, map, o)
#define DEC_GEN(DT, NPL)                                 \
    if (paged) DEC_GEN2(DT, NPL, true); else DEC_GEN2(DT, NPL, false)
        if (d->dtype == DM_F32) {
            if (npl == 1) DEC_GEN(DM_F32, 1); else if (npl == 2) DEC_GEN(DM_F32, 2); else DEC_GEN(DM_F32, 4);
        } else if (d->dtype == DM_BF16) {
            if (npl == 1) DEC_GEN(DM_BF16, 1); else if (npl == 2) DEC_GEN(DM_BF16, 2); else DEC_GEN(DM_BF16, 4);
        } else {
            if (npl == 1) DEC_GEN(DM_F16, 1); else if (npl == 2) DEC_GEN(DM_F16, 2); else DEC_GEN(DM_F16, 4);
        }
#undef DEC_GEN
#undef DEC_GEN2
        probe_add(DM_PROBE_ATTN_FWD_GENERIC);
        DM_LAUNCH_CHECK((opn + ": launch").c_str());
        return DM_OK;
    }
    const int nsplit = nsplit_of(d), span = span_of(d);
    if (nsplit > 4096) return refuse(opn + ": internal: more than 4096 splits");
    const size_t parts = (size_t)rows * nsplit;
    float *part_o = (float *)workspace;
    float *part_lse = (float *)((char *)workspace + align_up(parts * d->d * sizeof(float)));
    // the MFMA kernel's grid: key-value heads fastest (the heads of a split read neighbouring
    // bytes of the same cache rows at about the same time)
    dim3 grid_hf((unsigned)d->hkv, nsplit, (unsigned)d->b);
    const int g = (int)(d->hq / d->hkv);
#define DEC_MFMA2(DT, GG, PG, DD)                                                           \
    decode_split_mfma<DT, GG, PG, DD><<<grid_hf, 256, 0, st>>>(d->tk, d->hq, d->hkv, left, scale, \
                                                               nsplit, span, q, k, v, lengths, \
                                                               map, part_o, part_lse, o)
#define DEC_MFMA(DT, GG, DD)                         \
    if (paged) DEC_MFMA2(DT, GG, true, DD); else DEC_MFMA2(DT, GG, false, DD)
#define DEC_GM(DT, DD)                               \
    switch (g) {                                     \
        case 1: DEC_MFMA(DT, 1, DD); break;          \
        case 2: DEC_MFMA(DT, 2, DD); break;          \
        case 4: DEC_MFMA(DT, 4, DD); break;          \
        default: DEC_MFMA(DT, 8, DD); break;         \
    }
#define DEC_D(DT)                                    \
    switch (d->d) {                                  \
        case 64: DEC_GM(DT, 64); break;              \
        case 128: DEC_GM(DT, 128); break;            \
        default: DEC_GM(DT, 256); break;             \
    }
    {
        KernelTimer timer(DM_KERNEL_DECODE_SPLIT, st);
        if (d->dtype == DM_BF16) { DEC_D(DM_BF16); } else { DEC_D(DM_F16); }
    }
    if (nsplit > 1) {  // (one split: the split kernel wrote the output itself)
        KernelTimer timer(DM_KERNEL_DECODE_MERGE, st);
        if (d->dtype == DM_BF16) {
            decode_merge<DM_BF16><<<(unsigned)rows, 256, 0, st>>>(rows, d->d, nsplit, part_o, part_lse, o);
        } else {
            decode_merge<DM_F16><<<(unsigned)rows, 256, 0, st>>>(rows, d->d, nsplit, part_o, part_lse, o);
        }
    }
#undef DEC_D
#undef DEC_GM
#undef DEC_MFMA
#undef DEC_MFMA2
    probe_add(DM_PROBE_DECODE_SPLIT);
    if (nsplit > 1) probe_add(DM_PROBE_DECODE_MERGE);
    DM_LAUNCH_CHECK((opn + ": launch").c_str());
    return DM_OK;
}

// The split pass's workspace: partial outputs [B, Hq, nsplit, D] f32 and their log-sum-exps
// [B, Hq, nsplit].
static size_t decode_workspace(const dm_attention_desc *d, bool split) {
    if (!d || !split) return 0;
    const size_t parts = (size_t)(d->b * d->hq) * nsplit_of(d);
    return align_up(parts * d->d * sizeof(float)) + align_up(parts * sizeof(float));
}

// The no-allocation entry point's scratch: one array per device, held from the library's load
// until the process ends, for the split pass's partial outputs and log-sum-exps. Every call on a
// device shares it (calls that overlap on one device race). The split pass writes every partial
// it has, so nothing needs clearing between calls.
constexpr size_t kDecodeScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

// The device address of this device's `scratch`, looked up once per device (the array's name in
// host code is a host-side stand-in, never a device address).
static int scratch_address(void **out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void *addr[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "attention_decode_noalloc: hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return refuse("attention_decode_noalloc: device index " + std::to_string(dev) +
                      " beyond the library's table of " + std::to_string(kMaxDevices));
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess)
            return hip_status(e, "attention_decode_noalloc: hipGetSymbolAddress(scratch)");
        addr[dev] = p;
    }
    *out = addr[dev];
    return DM_OK;
}

}  // namespace dm

using namespace dm;

extern "C" {

size_t dm_attention_decode_workspace(const dm_attention_desc *d) {
    return d && d->hkv > 0 ? decode_workspace(d, split_takes(d)) : 0;
}

int dm_attention_decode(const dm_attention_desc *d, const void *q, const void *k, const void *v,
                        const int32_t *lengths, void *o, void *workspace, size_t workspace_bytes,
                        void *stream) {
    const char *op = "attention_decode";
    if (int rc = check_decode(op, d)) return rc;
    KvMap map = kv_strides(d, 0);
    if (d->cu_seqlens_k) {
        if (d->nseq != d->b)
            return refuse("attention_decode: a packed cache takes cu_seqlens_k [B + 1] with "
                          "nseq = B");
        map.offsets = d->cu_seqlens_k;
    }
    if (workspace_bytes < dm_attention_decode_workspace(d))
        return refuse("attention_decode: the workspace is smaller than dm_attention_decode_workspace");
    hipStream_t st = (hipStream_t)stream;
    const int64_t rows = d->b * d->hq;
    if (rows == 0 || d->d == 0) return DM_OK;
    if (d->tk == 0) {
        fill_zero(o, rows * d->d * dtype_bytes(d->dtype), st);
        DM_LAUNCH_CHECK("attention_decode: fill");
        return DM_OK;
    }
    const bool split = split_takes(d) && aligned_16b(q) && aligned_16b(k) && aligned_16b(v);
    return run_decode(op, d, split, false, q, k, v, lengths, map, o, workspace, st);
}

int dm_attention_decode_noalloc(const dm_attention_desc *d, const void *q, const void *k,
                                const void *v, const int32_t *lengths, void *o, void *stream) {
    if (int rc = check_decode("attention_decode", d)) return rc;
    const size_t need = dm_attention_decode_workspace(d);
    if (need > kDecodeScratchBytes)
        return refuse("attention_decode: the call needs " + std::to_string(need) +
                      " bytes of scratch, above the no-allocation entry point's " +
                      std::to_string(kDecodeScratchBytes) + "; use dm_attention_decode");
    void *ws = nullptr;
    if (need > 0)
        if (int rc = scratch_address(&ws)) return rc;
    return dm_attention_decode(d, q, k, v, lengths, o, ws, need, stream);
}

size_t dm_attention_decode_paged_workspace(const dm_attention_desc *d, int64_t page_size) {
    return d && d->hkv > 0 ? decode_workspace(d, paged_split_takes(d, page_size)) : 0;
}

int dm_attention_decode_paged(const dm_attention_desc *d, const void *q, const void *k_pages,
                              const void *v_pages, int64_t num_pages, int64_t page_size,
                              const int32_t *block_table, int64_t max_pages,
                              const int32_t *lengths, void *o, void *workspace,
                              size_t workspace_bytes, void *stream) {
    const char *op = "attention_decode_paged";
    if (int rc = check_decode(op, d)) return rc;
    if (page_size < 1 || max_pages < 0 || num_pages < 0)
        return refuse("attention_decode_paged: page_size must be positive, max_pages and "
                      "num_pages not negative");
    if (d->tk != max_pages * page_size)
        return refuse("attention_decode_paged: desc->tk (" + std::to_string(d->tk) +
                      ") must be max_pages * page_size (" + std::to_string(max_pages * page_size) +
                      ")");
    if (d->cu_seqlens_k)
        return refuse("attention_decode_paged: a paged cache takes a block table, not cu_seqlens_k");
    if (d->tk > 0 && d->b > 0 && !block_table)
        return refuse("attention_decode_paged: the block table is [B, max_pages] int32");
    if (workspace_bytes < dm_attention_decode_paged_workspace(d, page_size))
        return refuse("attention_decode_paged: the workspace is smaller than "
                      "dm_attention_decode_paged_workspace");
    hipStream_t st = (hipStream_t)stream;
    const int64_t rows = d->b * d->hq;
    if (rows == 0 || d->d == 0) return DM_OK;
    if (d->tk == 0) {
        fill_zero(o, rows * d->d * dtype_bytes(d->dtype), st);
        DM_LAUNCH_CHECK("attention_decode_paged: fill");
        return DM_OK;
    }
    KvMap map = kv_strides(d, page_size);
    map.block_table = block_table;
    map.page_size = page_size;
    map.max_pages = max_pages;
    map.num_pages = num_pages;
    const bool split = paged_split_takes(d, page_size) && aligned_16b(q) && aligned_16b(k_pages) &&
                       aligned_16b(v_pages);
    return run_decode(op, d, split, true, q, k_pages, v_pages, lengths, map, o, workspace, st);
}

}  // extern "C"
