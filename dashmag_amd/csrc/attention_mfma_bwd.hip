// MFMA attention backward for gfx950 (bf16/f16, head width 64, 128 or 256), deterministic: the
// query gradient is summed over the key tiles in a fixed order by its own sweep, as the
// reference's default does (crates/dash-ops/src/attention/kernels.rs:999-2058; the contract's
// `deterministic`, crates/dash-contract/src/attention.rs:100-105).
//
//   bwd_tiles  per tile of 32 query rows: the rows' visibility intervals, their union and the
//              keys every row sees.
//   bwd_dq     (head widths 64 and 128, first) per (tile of 128 queries, query head): delta =
//              rowsum(dO o O) from the dO it holds and each row's record (lse in log2 units, +inf
//              for a row that sees no key, delta, the interval) for the dK/dV kernel; then the
//              key tiles swept as the forward does, recomputing S^T and dP^T, dQ^T += K^T dS^T.
//   bwd_dkdv   per (tile of 128 keys, key-value head): sweeps the query heads of the group and
//              the 64-query tiles that see the keys. The keys and values stay in registers as the
//              B operands of S = Q K^T and dP = dO V^T (v_mfma_f32_32x32x16); P and dS go from the
//              products' output layout straight into the A operands of dV += P^T dO and
//              dK += dS^T Q, whose B operands come from transposed LDS copies of the tile.
//   bwd_dkdv_w4 (attention_bwd_w4.hip), bwd_dq_w4   head width 256: one wavefront per SIMD,
//              dV and dK in two passes
//              (work items of one launch), after bwd_prep (per query row: the interval, delta and
//              lse in log2 units).
#include <string>
#include <type_traits>

#include "attention_bwd.h"
#include "attention_kernels.h"
#include "mfma.h"

namespace dm {


// When there are few key blocks (a single long sequence), the dK/dV grid is too small to keep
// the chip busy and its causal work is uneven: the query heads of a group are then split over
// up to 4 workgroups per key block (at least two workgroups per compute unit), which write f32
// partials that a small kernel sums in a fixed order.
static int dkdv_hsplit(const dm_attention_desc *d) {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            n > 0)
            cus = n;
        else
            cus = 256;
    }
    const int64_t group = d->hq / d->hkv;
    const int64_t nwork = (d->tk + kKvBlock - 1) / kKvBlock * d->hkv * d->b;
    int split = 1;
    while (split < 4 && group % (2 * split) == 0 && nwork * split < 2 * cus) split *= 2;
    return split;
}

static size_t bwd_layout(const dm_attention_desc *d, char *base, BwdWs *w) {
    const int64_t rows = d->b * d->tq * d->hq, qrows = d->b * d->tq;
    const int64_t ntiles = (d->tq + kRowTile - 1) / kRowTile;
    size_t off = 0;
    auto take = [&](size_t bytes) -> char * {
        char *p = base ? base + off : nullptr;
        off += align_up(bytes);
        return p;
    };
    BwdWs x;
    x.lse2 = (float *)take(rows * 4);
    x.rec = (int4 *)take(rows * 16);
    x.rlo = (int32_t *)take(qrows * 4);
    x.rhi = (int32_t *)take(qrows * 4);
    x.trange = (int32_t *)take(d->b * ntiles * 4 * 4);
    x.hsplit = dkdv_hsplit(d);
    x.kvpart = x.hsplit > 1 ? (float *)take((size_t)x.hsplit * 2 * d->b * d->tk * d->hkv * d->d * 4)
                            : nullptr;
    const int64_t nkb = (d->tk + kKvBlock - 1) / kKvBlock;
    x.kbsteps = (int32_t *)take(d->b * (nkb + 1) * 4);
    x.order = (int32_t *)take(nkb * d->hkv * d->b * x.hsplit * (d->d == 256 ? 2 : 1) * 4);
    if (w) *w = x;
    return off;
}

// ------------------------------------------------------------------------------------------
// Prep
// ------------------------------------------------------------------------------------------

template <int DT, int D>
__global__ __launch_bounds__(256) void bwd_prep(MaskInfo m, int64_t B, int64_t Hq, AttnStrides sd,
                                                const uint16_t *__restrict__ o,
                                                const uint16_t *__restrict__ d_o,
                                                const float *__restrict__ lse,
                                                float *__restrict__ delta, BwdWs w) {
    // one wavefront per (b, query row); lanes over heads x D/8 chunks
    const int64_t Tq = m.tq;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;  // over B * Tq
    if (row >= B * Tq) return;
    const int64_t i = row % Tq, b = row / Tq;
    int64_t lo = 0, hi = 0;
    row_bounds(m, i, &lo, &hi);
    if (lane == 0) {
        w.rlo[row] = (int32_t)lo;
        w.rhi[row] = (int32_t)hi;
    }
    constexpr int CH = D / 8;       // 16-byte chunks per head row
    constexpr int HPI = 64 / CH;    // heads a wavefront covers at once
    constexpr int U = 8;            // rounds whose loads are issued together
    const int c = lane % CH;
    for (int64_t h0 = lane / CH; h0 < Hq; h0 += HPI * U) {
        uint4 a[U], g[U];
        float l[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t h = h0 + u * HPI;
            const bool ok = h < Hq;
            const int64_t hh = ok ? h : h0;
            a[u] = *(const uint4 *)(o + b * sd.o.b + i * sd.o.t + hh * sd.o.h + c * 8);
            g[u] = *(const uint4 *)(d_o + b * sd.g.b + i * sd.g.t + hh * sd.g.h + c * 8);
            l[u] = lse[row * Hq + hh];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t h = h0 + u * HPI;
            float s = unpack_lo<DT>(a[u].x) * unpack_lo<DT>(g[u].x) + unpack_hi<DT>(a[u].x) * unpack_hi<DT>(g[u].x) +
                      unpack_lo<DT>(a[u].y) * unpack_lo<DT>(g[u].y) + unpack_hi<DT>(a[u].y) * unpack_hi<DT>(g[u].y) +
                      unpack_lo<DT>(a[u].z) * unpack_lo<DT>(g[u].z) + unpack_hi<DT>(a[u].z) * unpack_hi<DT>(g[u].z) +
                      unpack_lo<DT>(a[u].w) * unpack_lo<DT>(g[u].w) + unpack_hi<DT>(a[u].w) * unpack_hi<DT>(g[u].w);
#pragma unroll
            for (int off = CH / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
            if (c == 0 && h < Hq) {
                const float l2 = l[u] == -INFINITY ? INFINITY : l[u] * 1.4426950408889634f;
                delta[row * Hq + h] = s;
                w.lse2[row * Hq + h] = l2;
                w.rec[row * Hq + h] = make_int4(__float_as_int(l2), __float_as_int(s), (int32_t)lo,
                                                (int32_t)(hi > lo ? hi - lo : 0));
            }
        }
    }
}

// Per tile of kRowTile rows: [union lo, union hi) of the rows' intervals, and [full lo, full hi), the
// keys every row of the tile sees (empty when a row of the tile sees nothing).
// ROWS (head widths 64 and 128, where no prep pass runs): the tile's rows' intervals are formed
// here and stored first (the dQ kernel forms delta and the rows' records itself).
template <bool ROWS>
__global__ __launch_bounds__(64) void bwd_tiles(MaskInfo m, int64_t B, int64_t Tq, BwdWs w) {
    const int64_t ntiles = (Tq + kRowTile - 1) / kRowTile;
    const int64_t t = blockIdx.x;
    if (t >= B * ntiles) return;
    const int64_t b = t / ntiles, tile = t % ntiles;
    const int64_t i = tile * kRowTile + threadIdx.x;
    int32_t ul = INT32_MAX, uh = INT32_MIN, fl = INT32_MIN, fh = INT32_MAX;
    if (threadIdx.x < kRowTile && i < Tq) {
        int32_t lo, hi;
        if constexpr (ROWS) {
            int64_t lo64 = 0, hi64 = 0;
            row_bounds(m, i, &lo64, &hi64);
            lo = (int32_t)lo64;
            hi = (int32_t)hi64;
            w.rlo[b * Tq + i] = lo;
            w.rhi[b * Tq + i] = hi;
        } else {
            lo = w.rlo[b * Tq + i];
            hi = w.rhi[b * Tq + i];
        }
        if (lo < hi) {
            ul = lo;
            uh = hi;
            fl = lo;
            fh = hi;
        } else {
            fl = INT32_MAX;
            fh = INT32_MIN;
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        ul = min(ul, __shfl_xor(ul, off, 64));
        uh = max(uh, __shfl_xor(uh, off, 64));
        fl = max(fl, __shfl_xor(fl, off, 64));
        fh = min(fh, __shfl_xor(fh, off, 64));
    }
    if (threadIdx.x == 0) {
        int32_t *r = w.trange + t * 4;
        r[0] = ul;
        r[1] = uh;
        r[2] = fl;
        r[3] = fh;
    }
}

// The dK/dV work list, longest first (a workgroup's time is its number of steps; running the
// longest first keeps the compute units evenly loaded to the end). One workgroup: per batch
// row, a difference array over the key blocks counts the tiles whose union interval reaches
// each block; the items are then placed by a counting sort on their step counts, descending.
// (Items with equal counts land in any order: the order only schedules, it does not change
// what a workgroup computes.)
constexpr int kOrderBuckets = 1024;
constexpr int kOrderLds = 8192;  // per-block counts held in LDS up to this many

// passes = 1: one work item per (key block, key-value head, query-head part), its steps the
// query tiles that see the block times the part's query heads. passes = 2 (the head width 256
// kernel): each of those twice, the dV pass first, then the dK pass, weighted by their products
// per step (2 : 3), and sorted together.
__global__ __launch_bounds__(1024) void bwd_order(int64_t B, int64_t Tq, int64_t Tk, int64_t Hkv,
                                                  int64_t group, int passes, BwdWs w) {
    __shared__ int32_t hist[kOrderBuckets];
    const int tid = threadIdx.x;
    const int64_t ntiles = (Tq + kRowTile - 1) / kRowTile;
    const int64_t nkb = (Tk + kKvBlock - 1) / kKvBlock;
    const int hs = w.hsplit;
    const int64_t per = group / hs;  // query heads per work item
    // difference array per batch row (in LDS when it fits), then its prefix sum, one wavefront
    // per batch row, 64 blocks at a time
    __shared__ int32_t cnt_lds[kOrderLds];
    const int64_t ncnt = B * (nkb + 1);
    int32_t *cnt = ncnt <= kOrderLds ? cnt_lds : w.kbsteps;
    for (int64_t x = tid; x < ncnt; x += 1024) cnt[x] = 0;
    __syncthreads();
    for (int64_t x = tid; x < B * ntiles; x += 1024) {
        const int64_t b = x / ntiles;
        const int32_t *r = w.trange + x * 4;
        if (r[0] < r[1]) {
            atomicAdd(&cnt[b * (nkb + 1) + r[0] / kKvBlock], 1);
            atomicAdd(&cnt[b * (nkb + 1) + (r[1] - 1) / kKvBlock + 1], -1);
        }
    }
    __syncthreads();
    {
        const int lane = tid & 63;
        for (int64_t b = tid >> 6; b < B; b += 16) {
            int32_t carry = 0;
            for (int64_t base = 0; base <= nkb; base += 64) {
                const int64_t kb = base + lane;
                int32_t x = kb <= nkb ? cnt[b * (nkb + 1) + kb] : 0;
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const int32_t y = __shfl_up(x, o, 64);
                    if (lane >= o) x += y;
                }
                if (kb <= nkb) cnt[b * (nkb + 1) + kb] = x + carry;
                carry += __shfl(x, 63, 64);
            }
        }
    }
    __syncthreads();
    // bucket = min(steps, kOrderBuckets - 1), steps = tiles x heads per item
    for (int x = tid; x < kOrderBuckets; x += 1024) hist[x] = 0;
    __syncthreads();
    const int64_t nwork = nkb * Hkv * B * hs;
    auto bucket = [&](int64_t item) {
        const int64_t weight = passes == 1 ? 1 : (item >= nwork ? 3 : 2);
        item = item % nwork;
        const int64_t kb = (item / (Hkv * hs)) % nkb, b = item / (Hkv * hs * nkb);
        const int64_t steps = (int64_t)cnt[b * (nkb + 1) + kb] * per * weight;
        return (int)(steps < kOrderBuckets - 1 ? steps : kOrderBuckets - 1);
    };
    const int64_t nitems = nwork * passes;
    for (int64_t x = tid; x < nitems; x += 1024) atomicAdd(&hist[bucket(x)], 1);
    __syncthreads();
    {
        // exclusive offsets, the largest bucket first: thread t takes bucket 1023 - t, a scan
        // within each wavefront, then over the wavefronts' totals
        static_assert(kOrderBuckets == 1024, "one bucket per thread");
        __shared__ int32_t wtot[16];
        const int lane = tid & 63, wv = tid >> 6;
        const int x = kOrderBuckets - 1 - tid;
        const int32_t c = hist[x];
        int32_t incl = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int32_t y = __shfl_up(incl, o, 64);
            if (lane >= o) incl += y;
        }
        if (lane == 63) wtot[wv] = incl;
        __syncthreads();
        int32_t before = 0;
        for (int u = 0; u < wv; u++) before += wtot[u];
        hist[x] = before + incl - c;
    }
    __syncthreads();
    for (int64_t x = tid; x < nitems; x += 1024) w.order[atomicAdd(&hist[bucket(x)], 1)] = (int32_t)x;

}

// ------------------------------------------------------------------------------------------
// dK, dV
// ------------------------------------------------------------------------------------------


// Wave pairs: a workgroup of 8 wavefronts takes 128 keys of one key-value head; wavefronts w and
// w + 4 (one SIMD) share the keys j0 + 32 w + [0, 32). Per 32-query step, wavefront w holds K
// and computes S = Q K^T, P = exp2(S c - lse2) (masked), hands P (f32) over through LDS and
// accumulates dV += P^T dO; wavefront w + 4 holds V and, one step behind, computes
// dP = dO V^T, dS = P (dP - delta) and accumulates dK += dS^T Q. The two halves carry equal
// MFMA work, and one's exp / pack work overlaps the other's products on the shared SIMD. All
// 512 threads stage Q / dO tiles from HBM two steps ahead through registers into three
// rotating LDS slots; one barrier per step.

#ifdef DM_TRACE_DKDV
// profiling aid (built only with -DDM_TRACE_DKDV): per-step clock stamps of one workgroup
__device__ uint64_t dm_trace[2][256][8];
#define DM_STAMP(role, step, k)                                                                  \
    do {                                                                                        \
        if (work == DM_TRACE_DKDV && kw == 0 && lane == 0 && (step) < 256)                      \
            dm_trace[role][step][k] = __builtin_readcyclecounter();                             \
    } while (0)
#else
#define DM_STAMP(role, step, k) \
    do {                        \
    } while (0)
#endif

template <int D>
struct DkdvSmem {
    DkdvSlot<D> slot[kDkdvSlots];
    float4 p[2][4][4][64];  // [step parity][key block][i / 4][lane]: P in the products' layout
    int4 sched[kDkdvRing];  // step k: {query head, tile, needs the mask, exists}
};

template <int DT, int D, bool PAD>
__global__ __launch_bounds__(512, 1) void bwd_dkdv(MaskInfo m, int64_t B, int64_t Hq,
                                                   int64_t Hkv, float scale, AttnStrides sd,
                                                   const uint16_t *__restrict__ q,
                                                   const uint16_t *__restrict__ k,
                                                   const uint16_t *__restrict__ v,
                                                   const uint16_t *__restrict__ d_o,
                                                   const float *__restrict__ delta,
                                                   BwdWs w, uint16_t *__restrict__ dk,
                                                   uint16_t *__restrict__ dv) {
    using Sm = DkdvSmem<D>;
    constexpr int RS = BwdStrides<D>::ROW, TS = BwdStrides<D>::TR;
    __shared__ Sm sm;
    constexpr int KSTEPS = D / 16, DT32 = D / 32;
    const int64_t Tq = m.tq, Tk = m.tk;
    const int64_t nkb = (Tk + kKvBlock - 1) / kKvBlock;
    const int hs = w.hsplit;
    const int64_t nwork = nkb * Hkv * B * hs;
    // the key-value head is the fastest index (an XCD holds one, with Hkv = 8), then the part of
    // the query heads, then the key block (the longest first under a causal mask)
    if ((int64_t)blockIdx.x >= nwork) return;
    const int64_t work = w.order[blockIdx.x];
    const int64_t kh = work % Hkv, part = (work / Hkv) % hs;
    const int64_t kb = (work / (Hkv * hs)) % nkb, b = work / (Hkv * hs * nkb);
    const int64_t group = Hq / Hkv;
    const int64_t h_first = kh * group + part * (group / hs);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool pwave = wave < 4;  // computes P and dV; the other half dS and dK
    const int kw = wave & 3;      // the key sub-block of this wavefront
    const int col = lane & 31, half = lane >> 5;
    const int32_t j0 = (int32_t)(kb * kKvBlock);
    const int32_t key = j0 + kw * 32 + col;  // this lane's key
    const bool kvalid = key < Tk;
    const bool kpad = PAD && kvalid && m.pad[b * Tk + key];
    const int32_t mkey = kpad ? -1 : key;  // a padded key is seen by no query (intervals >= 0)
    const float c2 = scale * 1.4426950408889634f;

    // K (P waves) or V (dS waves) of this lane's key as B operands (col = key, k = head dim)
    Frag8 bf[KSTEPS];
    {
        const uint16_t *bp = (pwave ? k + b * sd.k.b + (int64_t)key * sd.k.t + kh * sd.k.h
                                    : v + b * sd.v.b + (int64_t)key * sd.v.t + kh * sd.v.h) +
                             half * 8;
#pragma unroll
        for (int s = 0; s < KSTEPS; s++)
            bf[s].u = kvalid ? *(const uint4 *)(bp + s * 16) : make_uint4(0, 0, 0, 0);
    }
    // P waves accumulate dV, dS waves dK
    f32x16_t acc[DT32];
#pragma unroll
    for (int t = 0; t < DT32; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[t][i] = 0.f;

    const int64_t ntiles = (Tq + kDkdvStep - 1) / kDkdvStep;
    const int32_t *tr = w.trange + b * ntiles * 4;
    const int32_t j1 = j0 + kKvBlock < Tk ? j0 + kKvBlock : (int32_t)Tk;
    // The (head, tile) steps: the group's query heads, each over the tiles that see the keys.
    // A wavefront walks them 64 tiles at a time: one vector load of the tiles' ranges and two
    // ballots give the seeing tiles and the ones needing the per-element mask as bit masks, so
    // a step costs no memory round trip.
    const int32_t hend = (int32_t)(h_first + group / hs);
    struct TileIter {
        int32_t h, t;       // current step (h == hend: done)
        int32_t c0;         // first tile of the current 64-tile chunk
        uint64_t pending;   // seeing tiles of the chunk after t
        uint64_t cut;       // tiles of the chunk needing the per-element mask
        bool masked;        // whether step t needs it
    };
    auto scan = [&](TileIter &it) {
        const int32_t tt = it.c0 + lane;
        const int4 r = *(const int4 *)(tr + (tt < ntiles ? tt : ntiles - 1) * 4);
        const bool in = tt < ntiles;
        const bool see = in & (r.x < j1) & (r.y > j0);
        const bool part = PAD | (r.z > j0) | (r.w < j0 + kKvBlock);
        it.pending = __ballot(see);
        it.cut = __ballot(part);
    };
    // moves `it` to its next step (the first one when it.t < 0)
    auto next = [&](TileIter &it) {
        while (it.h < hend) {
            if (it.pending) {
                const int bit = __builtin_ctzll(it.pending);
                it.pending &= it.pending - 1;
                it.t = __builtin_amdgcn_readfirstlane(it.c0 + bit);
                it.masked = (it.cut >> bit) & 1;
                return;
            }
            it.c0 += 64;
            if (it.c0 >= ntiles) {
                it.h++;
                it.c0 = 0;
                if (it.h >= hend) return;
            }
            scan(it);
        }
    };
    auto start = [&](TileIter &it) {
        it.h = (int32_t)h_first;
        it.c0 = 0;
        it.t = -1;
        if (j0 >= Tk) {
            it.h = hend;
            return;
        }
        scan(it);
        next(it);
    };

    // staging: a step's Q and dO rows in 16-byte chunks (2 per thread) by buffer loads whose
    // range ends at the last query row, then a row copy and a transposed-read copy of each;
    // two register sets, a step's loads issued two steps before its store
    constexpr int CPR = D / 8, NCH = (kDkdvStep * CPR + 511) / 512, RSTEP = 512 / CPR;
    const int crow = tid / CPR, ccol = tid % CPR;  // crow >= kDkdvStep: no chunk (D = 64)
    // (row strides in bytes; the host checked that every byte range fits 32 bits)
    const uint32_t qrow_bytes = (uint32_t)(sd.q.t * 2), grow_bytes = (uint32_t)(sd.g.t * 2);
    const uint32_t qbytes = (uint32_t)(((Tq - 1) * sd.q.t + D) * 2);
    const uint32_t gbytes = (uint32_t)(((Tq - 1) * sd.g.t + D) * 2);
    struct Stage {
        uint4 q[NCH], g[NCH];
        uint4 rec;  // the row's lse2, delta, lo, hi - lo
    };
    Stage stg0, stg1;
    // Every call issues the same loads (so the compiler's count of loads in flight is exact and
    // a store waits only for its own set): rows past the tile's last valid row read zeros or a
    // repeated row, and every thread reads a row's lse / delta / interval (only 32 store them).
    // Zeros are harmless: a row whose interval is empty gets P = 0.
    const uint32_t rbytes = (uint32_t)(((Tq - 1) * Hq + 1) * 16);
    // each chunk's byte offset within a step's rows (loop-invariant)
    uint32_t qoff[NCH], goff[NCH];
#pragma unroll
    for (int u = 0; u < NCH; u++) {
        const uint32_t r = (uint32_t)((crow + u * RSTEP) & (kDkdvStep - 1));
        qoff[u] = r * qrow_bytes + ccol * 16;
        goff[u] = r * grow_bytes + ccol * 16;
    }
    auto load = [&](Stage &x, int64_t h, int64_t t) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t qrs = make_rsrc(q + b * sd.q.b + h * sd.q.h, qbytes);
        const __amdgpu_buffer_rsrc_t grs = make_rsrc(d_o + b * sd.g.b + h * sd.g.h, gbytes);
        const uint32_t i0 = (uint32_t)(t * kDkdvStep);
        const uint32_t qb = i0 * qrow_bytes, gb = i0 * grow_bytes;
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            x.q[u] = buf_load16(qrs, qb + qoff[u]);
            x.g[u] = buf_load16(grs, gb + goff[u]);
        }
        const uint32_t i = (uint32_t)(t * kDkdvStep) + (tid & (kDkdvStep - 1));
        const __amdgpu_buffer_rsrc_t rrs = make_rsrc(w.rec + b * Tq * Hq + h, rbytes);
        x.rec = buf_load16(rrs, i * (uint32_t)Hq * 16);
    };
    auto store = [&](const Stage &x, DkdvSlot<D> &sl) {
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            const int r = crow + u * RSTEP;
            if (r >= kDkdvStep) break;  // (head width 64: half the threads stage nothing)
            sl.q[r * (RS / 8) + ccol] = x.q[u];
            sl.qt[r * (TS / 8) + ccol] = x.q[u];
            sl.g[r * (RS / 8) + ccol] = x.g[u];
            sl.gt[r * (TS / 8) + ccol] = x.g[u];
        }
        if (tid < kDkdvStep) {
            sl.lse2[tid] = __uint_as_float(x.rec.x);
            sl.delta[tid] = __uint_as_float(x.rec.y);
            sl.rlo[tid] = (int32_t)x.rec.z;
            sl.rhi[tid] = (int32_t)x.rec.w;  // the span hi - lo
        }
    };

    // The schedule: wavefront 0 walks the steps and writes step k's entry into the ring
    // sm.sched five steps ahead of its use (entries 0 .. 4 up front, entry n + 5 in iteration
    // n); every wavefront reads the entries it needs, so a step costs the others no walk.
    TileIter it;
    auto publish = [&](const int k) __attribute__((always_inline)) {
        if (lane == 0)
            sm.sched[k % kDkdvRing] = make_int4(it.h, it.t, it.masked ? 1 : 0, it.h < hend ? 1 : 0);
        if (it.h < hend) next(it);
    };
    if (wave == 0) {
        start(it);
        for (int k = 0; k < 5; k++) publish(k);
    }
    __syncthreads();
    struct Entry {
        int32_t h, t;
        bool masked, valid;
    };
    auto entry = [&](const int k) __attribute__((always_inline)) -> Entry {
        const int4 e = sm.sched[k % kDkdvRing];
        Entry x;
        x.h = __builtin_amdgcn_readfirstlane(e.x);
        x.t = __builtin_amdgcn_readfirstlane(e.y);
        x.masked = __builtin_amdgcn_readfirstlane(e.z) != 0;
        x.valid = __builtin_amdgcn_readfirstlane(e.w) != 0;
        return x;
    };
    // prologue: step 0 into slot 0, steps 1 and 2 loading into the two register sets
    {
        const Entry e0 = entry(0), e1 = entry(1), e2 = entry(2);
        load(stg0, e0.valid ? e0.h : h_first, e0.valid ? e0.t : 0);
        if (e0.valid) store(stg0, sm.slot[0]);
        load(stg0, e1.valid ? e1.h : h_first, e1.valid ? e1.t : 0);
        load(stg1, e2.valid ? e2.h : h_first, e2.valid ? e2.t : 0);
    }
    __syncthreads();

    // stage step n + 1 (held by this step's register set) into slot `nslot`; the set then
    // loads step n + 3
    // (r1, r3: the schedule entries of steps n + 1 and n + 3, read by the caller before the
    // previous step's barrier, so their LDS latency hides behind it)
    auto restage = [&](const int n, const int nslot, Stage &x, const int4 r1, const int4 r3)
                       __attribute__((always_inline)) {
        const bool v1 = __builtin_amdgcn_readfirstlane(r1.w) != 0;
        Entry e;
        e.h = __builtin_amdgcn_readfirstlane(r3.x);
        e.t = __builtin_amdgcn_readfirstlane(r3.y);
        e.valid = __builtin_amdgcn_readfirstlane(r3.w) != 0;
        DM_STAMP(pwave ? 0 : 1, n, 4);
        if (v1) store(x, sm.slot[nslot]);
        DM_STAMP(pwave ? 0 : 1, n, 5);
        DM_STAMP(pwave ? 0 : 1, n, 6);
        // a step past the last loads the group's first tile again (the same loads every call)
        load(x, e.valid ? e.h : h_first, e.valid ? e.t : 0);
    };
    // P waves, step n: S = Q K^T, P (handed over in LDS), dV += P^T dO
    auto pstep = [&](const int n, const int cslot, const bool masked_flag)
                     __attribute__((always_inline)) {
        const DkdvSlot<D> &sl = sm.slot[cslot];
        const uint16_t *sq = (const uint16_t *)sl.q, *sgt = (const uint16_t *)sl.gt;
        f32x16_t s;
#pragma unroll
        for (int i = 0; i < 16; i++) s[i] = 0.f;
        const uint16_t *qa = sq + col * RS + half * 8;
#pragma unroll
        for (int st = 0; st < KSTEPS; st++) {
            Frag8 a;
            a.u = *(const uint4 *)(qa + st * 16);
            s = mfma32<DT>(a, bf[st], s);
        }
        // P = exp2(S c - lse2); element i is query 8 (i / 4) + 4 h + i % 4. The per-element
        // visibility test runs only on tiles the intervals cut (a branch around this VALU work
        // only; the products stay on one path)
        float p[16];
        auto probs = [&](auto cut_c) __attribute__((always_inline)) {
            constexpr bool CUT = decltype(cut_c)::value;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int r0 = j * 8 + half * 4;
                const float4 l4 = *(const float4 *)(sl.lse2 + r0);
                const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
                int lo4[4] = {0, 0, 0, 0}, hi4[4] = {0, 0, 0, 0};
                if constexpr (CUT) {
                    // rows hold lo and hi - lo: key visible iff (key - lo) < (hi - lo) unsigned
                    const int4 a4 = *(const int4 *)(sl.rlo + r0);
                    const int4 b4 = *(const int4 *)(sl.rhi + r0);
                    lo4[0] = a4.x; lo4[1] = a4.y; lo4[2] = a4.z; lo4[3] = a4.w;
                    hi4[0] = b4.x; hi4[1] = b4.y; hi4[2] = b4.z; hi4[3] = b4.w;
                }
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float x = fast_exp2(fmaf(s[4 * j + e], c2, -lv[e]));
                    if constexpr (CUT) {
                        const bool vis = (uint32_t)(mkey - lo4[e]) < (uint32_t)hi4[e];
                        x = vis ? x : 0.f;
                    }
                    p[4 * j + e] = x;
                }
            }
        };
        if (masked_flag)
            probs(std::true_type{});
        else
            probs(std::false_type{});
#pragma unroll
        for (int j = 0; j < 4; j++)
            sm.p[n & 1][kw][j][lane] =
                make_float4(p[4 * j], p[4 * j + 1], p[4 * j + 2], p[4 * j + 3]);
        DM_STAMP(0, n, 2);
        Frag8 pf[2];
#pragma unroll
        for (int u = 0; u < 2; u++)
            pf[u].u = make_uint4(pack2<DT>(p[8 * u], p[8 * u + 1]),
                                 pack2<DT>(p[8 * u + 2], p[8 * u + 3]),
                                 pack2<DT>(p[8 * u + 4], p[8 * u + 5]),
                                 pack2<DT>(p[8 * u + 6], p[8 * u + 7]));
        // dV += P^T dO: A = (row key, k = query) from the product's output, B = dO (k = query,
        // col = d) by transposed reads of the row-major tile
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int dt = 0; dt < DT32; dt++) {
                const Frag8 bg = lds_tr_frag(sgt, TS, u * 16, dt * 32, lane);
                acc[dt] = mfma32<DT>(pf[u], bg, acc[dt]);
            }
    };
    // dS waves, step m: dP = dO V^T, dS = P (dP - delta), dK += dS^T Q
    auto dsstep = [&](const int m, const int mslot) __attribute__((always_inline)) {
        const DkdvSlot<D> &sl = sm.slot[mslot];
        const uint16_t *sg = (const uint16_t *)sl.g, *sqt = (const uint16_t *)sl.qt;
        f32x16_t dp;
#pragma unroll
        for (int i = 0; i < 16; i++) dp[i] = 0.f;
        const uint16_t *ga = sg + col * RS + half * 8;
#pragma unroll
        for (int st = 0; st < KSTEPS; st++) {
            Frag8 a;
            a.u = *(const uint4 *)(ga + st * 16);
            dp = mfma32<DT>(a, bf[st], dp);
        }
        float ds[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float4 p4 = sm.p[m & 1][kw][j][lane];
            const float4 d4 = *(const float4 *)(sl.delta + j * 8 + half * 4);
            ds[4 * j + 0] = p4.x * (dp[4 * j + 0] - d4.x);
            ds[4 * j + 1] = p4.y * (dp[4 * j + 1] - d4.y);
            ds[4 * j + 2] = p4.z * (dp[4 * j + 2] - d4.z);
            ds[4 * j + 3] = p4.w * (dp[4 * j + 3] - d4.w);
        }
        DM_STAMP(1, m + 1, 2);
        Frag8 df[2];
#pragma unroll
        for (int u = 0; u < 2; u++)
            df[u].u = make_uint4(pack2<DT>(ds[8 * u], ds[8 * u + 1]),
                                 pack2<DT>(ds[8 * u + 2], ds[8 * u + 3]),
                                 pack2<DT>(ds[8 * u + 4], ds[8 * u + 5]),
                                 pack2<DT>(ds[8 * u + 6], ds[8 * u + 7]));
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int dt = 0; dt < DT32; dt++) {
                const Frag8 bq = lds_tr_frag(sqt, TS, u * 16, dt * 32, lane);
                acc[dt] = mfma32<DT>(df[u], bq, acc[dt]);
            }
    };

    // The steps run as iterations n = 0 .. N (N steps), one barrier each: the P waves compute
    // step n in iterations 0 .. N - 1, the dS waves step n - 1 in iterations 1 .. N. Each half
    // runs its own loop (the same barriers), unrolled by two so that each register set keeps
    // its own registers and its loads stay in flight across a step (a set chosen at run time
    // would be copied, and the copy waits for the loads).
    // slot indices rotate with n: cs = n % 3 (step n), ns = (n + 1) % 3, ps = (n + 2) % 3
    // = (n - 1) % 3
    int cs = 0, ns = 1, ps = 2;
    auto rotate = [&]() __attribute__((always_inline)) {
        const int t = ps;
        ps = cs;
        cs = ns;
        ns = t;
    };
    // The schedule entries a step needs (its own, and steps n + 1 and n + 3 for the staging)
    // are read at the end of the step before, ahead of its barrier: entry n + 4 was published
    // one step earlier, and the slots read are never the one wavefront 0 writes in that step.
    auto valid_of = [](const int4 e) { return __builtin_amdgcn_readfirstlane(e.w) != 0; };
    if (pwave) {
        int n = 0;
        int4 e0 = sm.sched[0], r1 = sm.sched[1], r3 = sm.sched[3];
        auto one = [&](Stage &x) __attribute__((always_inline)) {
            DM_STAMP(0, n, 0);
            restage(n, ns, x, r1, r3);
            DM_STAMP(0, n, 1);
            pstep(n, cs, __builtin_amdgcn_readfirstlane(e0.z) != 0);
            DM_STAMP(0, n, 3);
            if (wave == 0) publish(n + 5);
            e0 = r1;
            r1 = sm.sched[(n + 2) % kDkdvRing];
            r3 = sm.sched[(n + 4) % kDkdvRing];
            __syncthreads();
            n++;
            rotate();
        };
        for (;;) {
            if (!valid_of(e0)) break;
            one(stg0);
            if (!valid_of(e0)) break;
            one(stg1);
        }
        __syncthreads();  // iteration N
    } else {
        restage(0, ns, stg0, sm.sched[1], sm.sched[3]);
        __syncthreads();
        int n = 1;
        rotate();
        int4 em = sm.sched[0], r1 = sm.sched[2], r3 = sm.sched[4];
        auto one = [&](Stage &x) __attribute__((always_inline)) {
            DM_STAMP(1, n, 0);
            restage(n, ns, x, r1, r3);
            DM_STAMP(1, n, 1);
            dsstep(n - 1, ps);
            DM_STAMP(1, n, 3);
            em = sm.sched[n % kDkdvRing];
            r1 = sm.sched[(n + 2) % kDkdvRing];
            r3 = sm.sched[(n + 4) % kDkdvRing];
            __syncthreads();
            n++;
            rotate();
        };
        for (;;) {
            if (!valid_of(em)) break;
            one(stg1);
            if (!valid_of(em)) break;
            one(stg0);
        }
    }
    // write dV (P waves) or dK (scaled, dS waves): lane holds column d = 32 dt + col, rows =
    // keys 32 kw + 8 (i / 4) + 4 h + i % 4
    const float f = pwave ? 1.f : scale;
    if (hs == 1) {
        uint16_t *out = pwave ? dv : dk;
#pragma unroll
        for (int dt = 0; dt < DT32; dt++)
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                const int64_t ja = j0 + kw * 32 + (i / 4) * 8 + half * 4 + (i % 4);
                const uint32_t x2 = pack2<DT>(acc[dt][i] * f, acc[dt][i + 1] * f);
                const int64_t off = ((b * Tk + ja) * Hkv + kh) * D + dt * 32 + col;
                if (ja < Tk) out[off] = (uint16_t)(x2 & 0xffffu);
                if (ja + 1 < Tk) out[off + Hkv * D] = (uint16_t)(x2 >> 16);
            }
    } else {
        // f32 partial of this part: [part][dK = 0, dV = 1][B, Tk, Hkv, D]
        const int64_t n = B * Tk * Hkv * D;
        float *out = w.kvpart + (part * 2 + (pwave ? 1 : 0)) * n;
#pragma unroll
        for (int dt = 0; dt < DT32; dt++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int64_t ja = j0 + kw * 32 + (i / 4) * 8 + half * 4 + (i % 4);
                if (ja < Tk) out[((b * Tk + ja) * Hkv + kh) * D + dt * 32 + col] = acc[dt][i] * f;
            }
    }
}

// dK, dV = the sum of the parts' f32 partials, in part order, in the dtype.
template <int DT>
__global__ __launch_bounds__(256) void bwd_kv_reduce(int64_t n, int hs, const float *__restrict__ part,
                                                     uint16_t *__restrict__ dk,
                                                     uint16_t *__restrict__ dv) {
    const int64_t i4 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;  // 4 elements per thread
    if (i4 >= n) return;
#pragma unroll
    for (int which = 0; which < 2; which++) {
        float4 s = *(const float4 *)(part + which * n + i4);
        for (int p = 1; p < hs; p++) {
            const float4 x = *(const float4 *)(part + (p * 2 + which) * n + i4);
            s.x += x.x;
            s.y += x.y;
            s.z += x.z;
            s.w += x.w;
        }
        uint16_t *out = which ? dv : dk;
        *(uint2 *)(out + i4) = make_uint2(pack2<DT>(s.x, s.y), pack2<DT>(s.z, s.w));
    }
}

// ------------------------------------------------------------------------------------------
// dQ
// ------------------------------------------------------------------------------------------

#ifdef DM_TRACE_DQ
// profiling aid (built only with -DDM_TRACE_DQ=<workgroup>): per-step clock stamps of
// wavefronts 0 and 4 of one workgroup
__device__ uint64_t dm_trace_dq[2][256][4];
#define DM_QSTAMP(role, step, k)                                                                 \
    do {                                                                                        \
        if (blockIdx.x == (DM_TRACE_DQ) && (threadIdx.x & 255) == 0 && (step) < 256)            \
            dm_trace_dq[role][step][k] = __builtin_readcyclecounter();                          \
    } while (0)
extern "C" int dm_debug_trace_dq(void *host, size_t bytes) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(dm_trace_dq), bytes) == hipSuccess ? 0 : 1;
}
#else
#define DM_QSTAMP(role, step, k) \
    do {                         \
    } while (0)
#endif

// Wave pairs, as the dK/dV kernel: a workgroup of 8 wavefronts takes 128 queries of one query
// head; wavefronts w and w + 4 (one SIMD) share the queries 32 w + [0, 32). Per 32-key step,
// wavefront w holds Q and computes S^T = K Q^T and P (masked), handing P (f32) over through LDS;
// wavefront w + 4 holds dO and, one step behind, computes dP^T = V dO^T, dS = P (dP - delta)
// and accumulates dQ^T += K^T dS^T. Key / value tiles rotate through three LDS slots, staged
// two steps ahead through two register sets; one barrier per step.
constexpr int kDqStep = 32;  // keys per step

template <int D>
struct DqSlot {
    uint4 k[kDqStep * BwdStrides<D>::ROW / 8];
    uint4 kt[kDqStep * BwdStrides<D>::TR / 8];
    uint4 v[kDqStep * BwdStrides<D>::ROW / 8];
};

template <int D>
struct DqSmem {
    DqSlot<D> slot[3];
    float4 p[2][4][4][64];  // [step parity][query block][i / 4][lane]
    int32_t lo[4], hi[4], flo[4], fhi[4];
};

template <int DT, int D, bool PAD>
__global__ __launch_bounds__(512, 1) void bwd_dq(MaskInfo m, int64_t B, int64_t Hq, int64_t Hkv,
                                                 float scale, AttnStrides sd,
                                                 const uint16_t *__restrict__ q,
                                                 const uint16_t *__restrict__ k,
                                                 const uint16_t *__restrict__ v,
                                                 const uint16_t *__restrict__ d_o,
                                                 const uint16_t *__restrict__ o,
                                                 const float *__restrict__ lse,
                                                 float *__restrict__ delta, BwdWs w,
                                                 uint16_t *__restrict__ dq) {
    using Sm = DqSmem<D>;
    constexpr int RS = BwdStrides<D>::ROW, TS = BwdStrides<D>::TR;
    __shared__ Sm sm;
    constexpr int KSTEPS = D / 16, DT32 = D / 32;
    const int64_t Tq = m.tq, Tk = m.tk;
    const int64_t ntiles = (Tq + kDqM - 1) / kDqM;
    const int64_t nwork = ntiles * Hq * B;
    const int64_t work = blockIdx.x;
    if (work >= nwork) return;
    // the key-value head is the fastest index: consecutive blocks go to consecutive XCDs, so
    // an XCD (with Hkv = 8) holds one key-value head, whose keys and values stay in its L2,
    // and every XCD gets query tiles of every length (the longest first)
    const int64_t kh = work % Hkv;
    const int64_t h = kh * (Hq / Hkv) + (work / Hkv) % (Hq / Hkv);
    const int64_t tile = ntiles - 1 - (work / Hq) % ntiles;
    const int64_t b = work / (Hq * ntiles);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool pwave = wave < 4;  // computes P; the other half dS and dQ
    const int qw = wave & 3;      // the query block of this wavefront
    const int col = lane & 31, half = lane >> 5;
    const int64_t qi = tile * kDqM + qw * 32 + col;
    const bool qvalid = qi < Tq;
    int32_t lo = 0, hi = 0;
    float lse2 = INFINITY;
    if (qvalid) {
        lo = w.rlo[b * Tq + qi];
        hi = w.rhi[b * Tq + qi];
        // lse in log2 units, +inf for a row that sees no key (its probabilities are then 0)
        const float l = lse[(b * Tq + qi) * Hq + h];
        lse2 = l == -INFINITY ? INFINITY : l * 1.4426950408889634f;
    }
    const int32_t hi_row = hi;      // the row's interval, for its record
    if (lse2 == INFINITY) hi = lo;  // a query that sees no key: dq = 0
    if (pwave) {
        int32_t wl = lo < hi ? lo : INT32_MAX, wh = lo < hi ? hi : INT32_MIN;
        int32_t rfl = (qvalid && lo < hi) ? lo : (qvalid ? INT32_MAX : INT32_MIN);
        int32_t rfh = (qvalid && lo < hi) ? hi : (qvalid ? INT32_MIN : INT32_MAX);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            wl = min(wl, __shfl_xor(wl, off, 64));
            wh = max(wh, __shfl_xor(wh, off, 64));
            rfl = max(rfl, __shfl_xor(rfl, off, 64));
            rfh = min(rfh, __shfl_xor(rfh, off, 64));
        }
        if (lane == 0) {
            sm.lo[qw] = wl;
            sm.hi[qw] = wh;
            sm.flo[qw] = rfl;
            sm.fhi[qw] = rfh;
        }
    }
    __syncthreads();
    const int32_t kv_lo = min(min(sm.lo[0], sm.lo[1]), min(sm.lo[2], sm.lo[3]));
    const int32_t kv_hi = max(max(sm.hi[0], sm.hi[1]), max(sm.hi[2], sm.hi[3]));
    const int32_t span = hi - lo;  // visible iff (j - lo) < span, unsigned

    // Q (P waves) or dO (dS waves) of this lane's query as the B operand: col = query, k = d
    Frag8 bf[KSTEPS];
    {
        const uint16_t *src = (pwave ? q + b * sd.q.b + qi * sd.q.t + h * sd.q.h
                                     : d_o + b * sd.g.b + qi * sd.g.t + h * sd.g.h) +
                              half * 8;
#pragma unroll
        for (int s = 0; s < KSTEPS; s++)
            bf[s].u = qvalid ? *(const uint4 *)(src + s * 16) : make_uint4(0, 0, 0, 0);
    }
    // delta = rowsum(dO o O) for this query and head, by the dS wavefronts from the dO fragments
    // they hold (lane halves hold alternate 8-column pieces of the row); the O loads issue here,
    // beside dO's and the first tiles', and the sums are formed after the prologue. (Every lane
    // loads, a row past the end reading row 0, so the loads issue together without a branch
    // each; those lanes' sums are unused.)
    float dl = 0.f;
    uint4 ov[KSTEPS];
    if (!pwave) {
        const uint16_t *op = o + b * sd.o.b + (qvalid ? qi : 0) * sd.o.t + h * sd.o.h + half * 8;
#pragma unroll
        for (int s = 0; s < KSTEPS; s++) ov[s] = *(const uint4 *)(op + s * 16);
    }
    f32x16_t acc[DT32];
#pragma unroll
    for (int t = 0; t < DT32; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[t][i] = 0.f;
    const float c2 = scale * 1.4426950408889634f;
    const float nlse = -lse2;
    const int32_t kstride = (int32_t)sd.k.t, vstride = (int32_t)sd.v.t;
    const uint32_t kbytes = (uint32_t)(((Tk - 1) * sd.k.t + D) * 2);
    const uint32_t vbytes = (uint32_t)(((Tk - 1) * sd.v.t + D) * 2);
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(k + b * sd.k.b + kh * sd.k.h, kbytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(v + b * sd.v.b + kh * sd.v.h, vbytes);
    const uint8_t *pad = PAD ? m.pad + b * Tk : nullptr;

    // staging: a tile's K and V rows in 16-byte chunks over the 512 threads, two register
    // sets, every call the same loads (tiles past the range re-read the first)
    constexpr int CPR = D / 8, NCH = (kDqStep * CPR + 511) / 512, RSTEP = 512 / CPR;
    const int crow = tid / CPR, ccol = tid % CPR;  // crow >= kDqStep: no chunk (D = 64)
    struct KvStage {
        uint4 k[NCH], v[NCH];
    };
    KvStage st0, st1;
    const int nsteps = kv_lo < kv_hi ? (kv_hi - kv_lo + kDqStep - 1) / kDqStep : 0;
    uint32_t koff[NCH], voff[NCH];  // each chunk's byte offset within a step's rows
#pragma unroll
    for (int u = 0; u < NCH; u++) {
        const int r = (crow + u * RSTEP) & (kDqStep - 1);
        koff[u] = (uint32_t)(r * kstride + ccol * 8) * 2;
        voff[u] = (uint32_t)(r * vstride + ccol * 8) * 2;
    }
    auto load = [&](KvStage &x, int n) __attribute__((always_inline)) {
        const int32_t j0 = kv_lo + (n < nsteps ? n : 0) * kDqStep;
        const uint32_t kb = (uint32_t)(j0 * kstride) * 2, vb = (uint32_t)(j0 * vstride) * 2;
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            x.k[u] = buf_load16(krs, kb + koff[u]);
            x.v[u] = buf_load16(vrs, vb + voff[u]);
        }
    };
    auto store = [&](const KvStage &x, DqSlot<D> &sl) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            const int r = crow + u * RSTEP;
            if (r >= kDqStep) break;
            sl.k[r * (RS / 8) + ccol] = x.k[u];
            sl.kt[r * (TS / 8) + ccol] = x.k[u];
            sl.v[r * (RS / 8) + ccol] = x.v[u];
        }
    };

    // P waves, step n (keys j0 = kv_lo + 32 n): S^T = K Q^T, P into LDS
    auto pstep = [&](const int n, const int cslot) __attribute__((always_inline)) {
        const int32_t j0 = kv_lo + n * kDqStep;
        const uint16_t *ka = (const uint16_t *)sm.slot[cslot].k + col * RS + half * 8;
        f32x16_t s;
#pragma unroll
        for (int i = 0; i < 16; i++) s[i] = 0.f;
#pragma unroll
        for (int st = 0; st < KSTEPS; st++) {
            Frag8 a;
            a.u = *(const uint4 *)(ka + st * 16);
            s = mfma32<DT>(a, bf[st], s);
        }
        // element i is key j0 + 8 (i / 4) + 4 h + i % 4
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            float p4[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int i = 4 * jj + e;
                const int32_t j = j0 + jj * 8 + half * 4 + e;
                float x = fast_exp2(fmaf(s[i], c2, nlse));
                bool vis = (uint32_t)(j - lo) < (uint32_t)span;
                if constexpr (PAD) vis = vis & (pad[j < Tk ? j : Tk - 1] == 0);
                p4[e] = vis ? x : 0.f;
            }
            sm.p[n & 1][qw][jj][lane] = make_float4(p4[0], p4[1], p4[2], p4[3]);
        }
    };
    // dS waves, step m: dP^T = V dO^T, dS = P (dP - delta), dQ^T += K^T dS^T
    auto dsstep = [&](const int m, const int mslot) __attribute__((always_inline)) {
        const DqSlot<D> &sl = sm.slot[mslot];
        const uint16_t *va = (const uint16_t *)sl.v + col * RS + half * 8;
        const uint16_t *skt = (const uint16_t *)sl.kt;
        f32x16_t dp;
#pragma unroll
        for (int i = 0; i < 16; i++) dp[i] = 0.f;
#pragma unroll
        for (int st = 0; st < KSTEPS; st++) {
            Frag8 a;
            a.u = *(const uint4 *)(va + st * 16);
            dp = mfma32<DT>(a, bf[st], dp);
        }
        float ds[16];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const float4 p4 = sm.p[m & 1][qw][jj][lane];
            ds[4 * jj + 0] = p4.x * (dp[4 * jj + 0] - dl);
            ds[4 * jj + 1] = p4.y * (dp[4 * jj + 1] - dl);
            ds[4 * jj + 2] = p4.z * (dp[4 * jj + 2] - dl);
            ds[4 * jj + 3] = p4.w * (dp[4 * jj + 3] - dl);
        }
        Frag8 df[2];
#pragma unroll
        for (int u = 0; u < 2; u++)
            df[u].u = make_uint4(pack2<DT>(ds[8 * u], ds[8 * u + 1]),
                                 pack2<DT>(ds[8 * u + 2], ds[8 * u + 3]),
                                 pack2<DT>(ds[8 * u + 4], ds[8 * u + 5]),
                                 pack2<DT>(ds[8 * u + 6], ds[8 * u + 7]));
        // A = K^T by transposed reads of the row-major K tile
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int dt = 0; dt < DT32; dt++) {
                const Frag8 a = lds_tr_frag(skt, TS, u * 16, dt * 32, lane);
                acc[dt] = mfma32<DT>(a, df[u], acc[dt]);
            }
    };

    // prologue: step 0 into slot 0, steps 1 and 2 loading into the two register sets
    load(st0, 0);
    if (nsteps > 0) store(st0, sm.slot[0]);
    load(st0, 1);
    load(st1, 2);
    if (!pwave) {
        // delta (the row's record for the dK/dV kernel, which runs after this one, is stored at
        // the end)
        float acc_d = 0.f;
#pragma unroll
        for (int s = 0; s < KSTEPS; s++) {
            const uint32_t ow[4] = {ov[s].x, ov[s].y, ov[s].z, ov[s].w};
            const uint32_t gw[4] = {bf[s].u.x, bf[s].u.y, bf[s].u.z, bf[s].u.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                acc_d = fmaf(unpack_lo<DT>(ow[e]), unpack_lo<DT>(gw[e]), acc_d);
                acc_d = fmaf(unpack_hi<DT>(ow[e]), unpack_hi<DT>(gw[e]), acc_d);
            }
        }
        dl = acc_d + __shfl_xor(acc_d, 32, 64);
    }
    __syncthreads();
    // iterations n = 0 .. nsteps: the P waves compute step n (n < nsteps), the dS waves step
    // n - 1 (n >= 1); each iteration stores step n + 1 from its set and loads step n + 3
    int cs = 0, ns = 1, ps = 2;
    auto rotate = [&]() __attribute__((always_inline)) {
        const int t = ps;
        ps = cs;
        cs = ns;
        ns = t;
    };
    auto restage = [&](const int n, KvStage &x) __attribute__((always_inline)) {
        if (n + 1 < nsteps) store(x, sm.slot[ns]);
        load(x, n + 3);
    };
    if (pwave) {
        int n = 0;
        // (both halves run on every pass, the second computing nothing past the last step: on
        // every path through the loop the second register set's loads are then the most recent,
        // and the compiler's wait counts keep them in flight across a step)
        auto one = [&](KvStage &x) __attribute__((always_inline)) {
            DM_QSTAMP(0, n, 0);
            restage(n, x);
            DM_QSTAMP(0, n, 1);
            if (n < nsteps) pstep(n, cs);
            DM_QSTAMP(0, n, 2);
            __syncthreads();
            n++;
            rotate();
        };
        while (n < nsteps) {
            one(st0);
            one(st1);
        }
        __syncthreads();  // the dS waves' last iteration
    } else {
        restage(0, st0);
        __syncthreads();
        int n = 1;
        rotate();
        auto one = [&](KvStage &x) __attribute__((always_inline)) {
            DM_QSTAMP(1, n, 0);
            restage(n, x);
            DM_QSTAMP(1, n, 1);
            if (n <= nsteps) dsstep(n - 1, ps);
            DM_QSTAMP(1, n, 2);
            __syncthreads();
            n++;
            rotate();
        };
        while (n <= nsteps) {
            one(st1);
            one(st0);
        }
        // the row's record for the dK/dV kernel, stored at the end so that the loop's waits for
        // its loads do not also wait for these stores
        if (qvalid && half == 0) {
            const int64_t r = (b * Tq + qi) * Hq + h;
            w.rec[r] = make_int4(__float_as_int(lse2), __float_as_int(dl), lo, hi_row > lo ? hi_row - lo : 0);
        }
        if (qvalid) {
            uint16_t *op = dq + ((b * Tq + qi) * Hq + h) * D;
#pragma unroll
            for (int dt = 0; dt < DT32; dt++)
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    const int d = dt * 32 + g4 * 8 + half * 4;
                    uint2 wv;
                    wv.x = pack2<DT>(acc[dt][g4 * 4 + 0] * scale, acc[dt][g4 * 4 + 1] * scale);
                    wv.y = pack2<DT>(acc[dt][g4 * 4 + 2] * scale, acc[dt][g4 * 4 + 3] * scale);
                    *(uint2 *)(op + d) = wv;
                }
        }
    }
}

// dQ at D = 256: 4 wavefronts of 32 queries (128 per workgroup), each holding its queries' Q
// and dO fragments and dQ^T (256 x 32) over the key steps: S^T = K Q^T, dP^T = V dO^T,
// dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T (48 products per 32-key step). Key and value tiles
// rotate through two LDS slots, staged one step ahead.
template <int D>
struct Dq4Smem {
    DqSlot<D> slot[2];
    int32_t lo[4], hi[4];
};

template <int DT, int D, bool PAD>
__global__ __launch_bounds__(256, 1) void bwd_dq_w4(MaskInfo m, int64_t B, int64_t Hq, int64_t Hkv,
                                                    float scale, AttnStrides sd,
                                                    const uint16_t *__restrict__ q,
                                                    const uint16_t *__restrict__ k,
                                                    const uint16_t *__restrict__ v,
                                                    const uint16_t *__restrict__ d_o,
                                                    const float *__restrict__ delta, BwdWs w,
                                                    uint16_t *__restrict__ dq) {
    constexpr int RS = BwdStrides<D>::ROW, TS = BwdStrides<D>::TR;
    __shared__ Dq4Smem<D> sm;
    constexpr int KSTEPS = D / 16, DT32 = D / 32;
    const int64_t Tq = m.tq, Tk = m.tk;
    const int64_t ntiles = (Tq + kDqM - 1) / kDqM;
    const int64_t nwork = ntiles * Hq * B;
    const int64_t work = blockIdx.x;
    if (work >= nwork) return;
    const int64_t kh = work % Hkv;
    const int64_t h = kh * (Hq / Hkv) + (work / Hkv) % (Hq / Hkv);
    const int64_t tile = ntiles - 1 - (work / Hq) % ntiles;
    const int64_t b = work / (Hq * ntiles);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, half = lane >> 5;
    const int64_t qi = tile * kDqM + wave * 32 + col;
    const bool qvalid = qi < Tq;
    int32_t lo = 0, hi = 0;
    float lse2 = INFINITY, dl = 0.f;
    if (qvalid) {
        lo = w.rlo[b * Tq + qi];
        hi = w.rhi[b * Tq + qi];
        lse2 = w.lse2[(b * Tq + qi) * Hq + h];
        dl = delta[(b * Tq + qi) * Hq + h];
    }
    if (lse2 == INFINITY) hi = lo;  // a query that sees no key: dq = 0
    {
        int32_t wl = lo < hi ? lo : INT32_MAX, wh = lo < hi ? hi : INT32_MIN;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            wl = min(wl, __shfl_xor(wl, off, 64));
            wh = max(wh, __shfl_xor(wh, off, 64));
        }
        if (lane == 0) {
            sm.lo[wave] = wl;
            sm.hi[wave] = wh;
        }
    }
    __syncthreads();
    const int32_t kv_lo = min(min(sm.lo[0], sm.lo[1]), min(sm.lo[2], sm.lo[3]));
    const int32_t kv_hi = max(max(sm.hi[0], sm.hi[1]), max(sm.hi[2], sm.hi[3]));
    const int32_t span = hi - lo;

    Frag8 qf[KSTEPS], gf[KSTEPS];  // B operands: col = query, k = d
    {
        const uint16_t *qp = q + b * sd.q.b + qi * sd.q.t + h * sd.q.h + half * 8;
        const uint16_t *gp = d_o + b * sd.g.b + qi * sd.g.t + h * sd.g.h + half * 8;
#pragma unroll
        for (int st = 0; st < KSTEPS; st++) {
            qf[st].u = qvalid ? *(const uint4 *)(qp + st * 16) : make_uint4(0, 0, 0, 0);
            gf[st].u = qvalid ? *(const uint4 *)(gp + st * 16) : make_uint4(0, 0, 0, 0);
        }
    }
    f32x16_t acc[DT32];
#pragma unroll
    for (int t = 0; t < DT32; t++) acc[t] = zero16();
    const float c2 = scale * 1.4426950408889634f;
    const float nlse = -lse2;
    const int32_t kstride = (int32_t)sd.k.t, vstride = (int32_t)sd.v.t;
    const uint32_t kbytes = (uint32_t)(((Tk - 1) * sd.k.t + D) * 2);
    const uint32_t vbytes = (uint32_t)(((Tk - 1) * sd.v.t + D) * 2);
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(k + b * sd.k.b + kh * sd.k.h, kbytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(v + b * sd.v.b + kh * sd.v.h, vbytes);
    const uint8_t *pad = PAD ? m.pad + b * Tk : nullptr;

    constexpr int CPR = D / 8, NCH = kDqStep * CPR / 256, RSTEP = 256 / CPR;
    const int crow = tid / CPR, ccol = tid % CPR;
    uint32_t koff[NCH], voff[NCH];
#pragma unroll
    for (int u = 0; u < NCH; u++) {
        const int r = crow + u * RSTEP;
        koff[u] = (uint32_t)(r * kstride + ccol * 8) * 2;
        voff[u] = (uint32_t)(r * vstride + ccol * 8) * 2;
    }
    struct KvStage {
        uint4 k[NCH], v[NCH];
    };
    KvStage stg;
    const int nsteps = kv_lo < kv_hi ? (kv_hi - kv_lo + kDqStep - 1) / kDqStep : 0;
    auto load = [&](int n) __attribute__((always_inline)) {
        const int32_t jj = kv_lo + (n < nsteps ? n : 0) * kDqStep;
        const uint32_t kb = (uint32_t)(jj * kstride) * 2, vb = (uint32_t)(jj * vstride) * 2;
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            stg.k[u] = buf_load16(krs, kb + koff[u]);
            stg.v[u] = buf_load16(vrs, vb + voff[u]);
        }
    };
    auto store = [&](DqSlot<D> &sl) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            const int r = crow + u * RSTEP;
            sl.k[r * (RS / 8) + ccol] = stg.k[u];
            sl.kt[r * (TS / 8) + ccol] = stg.k[u];
            sl.v[r * (RS / 8) + ccol] = stg.v[u];
        }
    };
    auto step = [&](const int n, const DqSlot<D> &sl) __attribute__((always_inline)) {
        const int32_t jb = kv_lo + n * kDqStep;
        const uint16_t *ka = (const uint16_t *)sl.k + col * RS + half * 8;
        const uint16_t *va = (const uint16_t *)sl.v + col * RS + half * 8;
        f32x16_t s = zero16(), dp = zero16();
#pragma unroll
        for (int st = 0; st < KSTEPS; st++) {
            Frag8 a;
            a.u = *(const uint4 *)(ka + st * 16);
            s = mfma32<DT>(a, qf[st], s);
        }
#pragma unroll
        for (int st = 0; st < KSTEPS; st++) {
            Frag8 a;
            a.u = *(const uint4 *)(va + st * 16);
            dp = mfma32<DT>(a, gf[st], dp);
        }
        // element i is key jb + 8 (i / 4) + 4 h + i % 4
        float ds[16];
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int i = 4 * jj + e;
                const int32_t j = jb + jj * 8 + half * 4 + e;
                float x = fast_exp2(fmaf(s[i], c2, nlse));
                bool vis = (uint32_t)(j - lo) < (uint32_t)span;
                if constexpr (PAD) vis = vis & (pad[j < Tk ? j : Tk - 1] == 0);
                ds[i] = vis ? x * (dp[i] - dl) : 0.f;
            }
        Frag8 df[2];
#pragma unroll
        for (int u = 0; u < 2; u++)
            df[u].u = make_uint4(pack2<DT>(ds[8 * u], ds[8 * u + 1]), pack2<DT>(ds[8 * u + 2], ds[8 * u + 3]),
                                 pack2<DT>(ds[8 * u + 4], ds[8 * u + 5]), pack2<DT>(ds[8 * u + 6], ds[8 * u + 7]));
        const uint16_t *skt = (const uint16_t *)sl.kt;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int dt = 0; dt < DT32; dt++)
                acc[dt] = mfma32<DT>(lds_tr_frag(skt, TS, u * 16, dt * 32, lane), df[u], acc[dt]);
    };
    load(0);
    if (nsteps > 0) store(sm.slot[0]);
    load(1);
    __syncthreads();
    for (int n = 0; n < nsteps; n++) {
        if (n + 1 < nsteps) store(sm.slot[(n + 1) & 1]);
        load(n + 2);
        step(n, sm.slot[n & 1]);
        __syncthreads();
    }
    if (qvalid) {
        uint16_t *op = dq + ((b * Tq + qi) * Hq + h) * D;
#pragma unroll
        for (int dt = 0; dt < DT32; dt++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const int d = dt * 32 + g4 * 8 + half * 4;
                uint2 wv;
                wv.x = pack2<DT>(acc[dt][g4 * 4 + 0] * scale, acc[dt][g4 * 4 + 1] * scale);
                wv.y = pack2<DT>(acc[dt][g4 * 4 + 2] * scale, acc[dt][g4 * 4 + 3] * scale);
                *(uint2 *)(op + d) = wv;
            }
    }
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------

// The shapes and strides the MFMA backward takes (its buffer loads use 32-bit byte offsets
// from one (batch row, head) base; 16-byte vector loads need 16-byte rows).
static bool mfma_bwd_shape_takes(const dm_attention_desc *d) {
    const AttnStrides s = attn_strides(d);
    return (d->dtype == DM_BF16 || d->dtype == DM_F16) &&
           (d->d == 64 || d->d == 128 || d->d == 256) && d->tq < (1ll << 30) && d->tk < (1ll << 30) && scale_of(d) > 0.f &&
           rows_fit_32bit(s.k, d->tk, d->d) && rows_fit_32bit(s.v, d->tk, d->d) &&
           rows_fit_32bit(s.q, d->tq, d->d) && rows_fit_32bit(s.g, d->tq, d->d) &&
           d->tq * d->hq < (1ll << 28) && strides_16b(s.q) && strides_16b(s.k) &&
           strides_16b(s.v) && strides_16b(s.o) && strides_16b(s.g);
}

bool mfma_bwd_takes(const dm_attention_desc *d, const void *q, const void *k, const void *v,
                    const void *o, const void *d_o) {
    return mfma_bwd_shape_takes(d) && aligned_16b(q) && aligned_16b(k) && aligned_16b(v) &&
           aligned_16b(o) && aligned_16b(d_o);
}

size_t mfma_bwd_workspace(const dm_attention_desc *d) {
    return mfma_bwd_shape_takes(d) ? bwd_layout(d, nullptr, nullptr) : 0;
}

#ifdef DM_TRACE_DKDV
extern "C" int dm_debug_trace(void *host, size_t bytes) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(dm_trace), bytes) == hipSuccess ? 0 : 1;
}
#endif

int launch_attn_bwd_mfma(const MaskInfo &m, const dm_attention_desc *d, float scale,
                         const void *q, const void *k, const void *v, const void *o,
                         const float *lse, const void *d_o, void *dq, void *dk, void *dv,
                         float *delta, void *workspace, hipStream_t st) {
    BwdWs w;
    bwd_layout(d, (char *)workspace, &w);
    const int64_t qrows = d->b * d->tq;
    const int64_t ntiles_r = (d->tq + kRowTile - 1) / kRowTile;
    const int64_t nkb = (d->tk + kKvBlock - 1) / kKvBlock;
    const int64_t nq = (d->tq + kDqM - 1) / kDqM;
    const int64_t nb_kv = nkb * d->hkv * d->b * w.hsplit;
    const int64_t nb_q = nq * d->hq * d->b;
    if (2 * nb_kv >= (1ll << 31) || nb_q >= (1ll << 31)) return refuse("attention_backward: too large");
    const uint16_t *qq = (const uint16_t *)q, *kk = (const uint16_t *)k, *vv = (const uint16_t *)v;
    const uint16_t *oo = (const uint16_t *)o, *gg = (const uint16_t *)d_o;
    const AttnStrides sd = attn_strides(d);
#define BWD(DT, DD)                                                                            \
    bwd_tiles<true><<<(unsigned)(d->b * ntiles_r), 64, 0, st>>>(m, d->b, d->tq, w);            \
    bwd_order<<<1, 1024, 0, st>>>(d->b, d->tq, d->tk, d->hkv, d->hq / d->hkv, 1, w);           \
    if (m.pad) {                                                                               \
        { KernelTimer t2(DM_KERNEL_ATTN_BWD_DQ, st);                                         \
        bwd_dq<DT, DD, true><<<(unsigned)nb_q, 512, 0, st>>>(m, d->b, d->hq, d->hkv, scale, sd, \
                                                             qq, kk, vv, gg, oo, lse, delta, w, \
                                                             (uint16_t *)dq); }                \
        { KernelTimer t1(DM_KERNEL_ATTN_BWD_DKDV, st);                                       \
        bwd_dkdv<DT, DD, true><<<(unsigned)nb_kv, 512, 0, st>>>(m, d->b, d->hq, d->hkv, scale, \
                                                                sd, qq, kk, vv, gg, delta, w,      \
                                                                (uint16_t *)dk, (uint16_t *)dv); } \
    } else {                                                                                   \
        { KernelTimer t2(DM_KERNEL_ATTN_BWD_DQ, st);                                         \
        bwd_dq<DT, DD, false><<<(unsigned)nb_q, 512, 0, st>>>(m, d->b, d->hq, d->hkv, scale, sd, \
                                                              qq, kk, vv, gg, oo, lse, delta, w, \
                                                              (uint16_t *)dq); }               \
        { KernelTimer t1(DM_KERNEL_ATTN_BWD_DKDV, st);                                       \
        bwd_dkdv<DT, DD, false><<<(unsigned)nb_kv, 512, 0, st>>>(m, d->b, d->hq, d->hkv, scale, \
                                                                 sd, qq, kk, vv, gg, delta, w,     \
                                                                 (uint16_t *)dk, (uint16_t *)dv); } \
    }
#define DKDV4(DT, P)                                                                           \
    launch_dkdv_w4(DT, P, nb_kv, m, d->b, d->hq, d->hkv, scale, sd, qq, kk, vv, gg, delta, w,   \
                   (uint16_t *)dk, (uint16_t *)dv, st)
#define BWD4(DT)                                                                               \
    bwd_prep<DT, 256><<<(unsigned)((qrows + 3) / 4), 256, 0, st>>>(m, d->b, d->hq, sd, oo, gg, \
                                                                    lse, delta, w);            \
    bwd_tiles<false><<<(unsigned)(d->b * ntiles_r), 64, 0, st>>>(m, d->b, d->tq, w);           \
    bwd_order<<<1, 1024, 0, st>>>(d->b, d->tq, d->tk, d->hkv, d->hq / d->hkv, 2, w);           \
    if (m.pad) {                                                                               \
        { KernelTimer t1(DM_KERNEL_ATTN_BWD_DKDV, st);                                       \
          DKDV4(DT, true); }                                                                   \
        { KernelTimer t2(DM_KERNEL_ATTN_BWD_DQ, st);                                         \
        bwd_dq_w4<DT, 256, true><<<(unsigned)nb_q, 256, 0, st>>>(                             \
            m, d->b, d->hq, d->hkv, scale, sd, qq, kk, vv, gg, delta, w, (uint16_t *)dq); }    \
    } else {                                                                                   \
        { KernelTimer t1(DM_KERNEL_ATTN_BWD_DKDV, st);                                       \
          DKDV4(DT, false); }                                                                  \
        { KernelTimer t2(DM_KERNEL_ATTN_BWD_DQ, st);                                         \
        bwd_dq_w4<DT, 256, false><<<(unsigned)nb_q, 256, 0, st>>>(                            \
            m, d->b, d->hq, d->hkv, scale, sd, qq, kk, vv, gg, delta, w, (uint16_t *)dq); }    \
    }
    if (d->dtype == DM_BF16) {
        if (d->d == 64) { BWD(DM_BF16, 64); } else if (d->d == 128) { BWD(DM_BF16, 128); } else { BWD4(DM_BF16); }
    } else {
        if (d->d == 64) { BWD(DM_F16, 64); } else if (d->d == 128) { BWD(DM_F16, 128); } else { BWD4(DM_F16); }
    }
#undef BWD
#undef BWD4
#undef DKDV4
    if (w.hsplit > 1) {
        const int64_t n = d->b * d->tk * d->hkv * d->d;  // a multiple of 4 (D is 64, 128 or 256)
        const unsigned blocks = (unsigned)((n / 4 + 255) / 256);
        if (d->dtype == DM_BF16)
            bwd_kv_reduce<DM_BF16><<<blocks, 256, 0, st>>>(n, w.hsplit, w.kvpart, (uint16_t *)dk,
                                                         (uint16_t *)dv);
        else
            bwd_kv_reduce<DM_F16><<<blocks, 256, 0, st>>>(n, w.hsplit, w.kvpart, (uint16_t *)dk,
                                                        (uint16_t *)dv);
    }
    probe_add(DM_PROBE_ATTN_BWD_MFMA, 4);
    DM_LAUNCH_CHECK("attention_backward: MFMA launch");
    return DM_OK;
}

}  // namespace dm
