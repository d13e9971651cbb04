// MFMA attention for gfx950: bf16/f16 inputs, f32 accumulation, head width 64 or 128.
//
// Forward (the flash-attention forward of crates/dash-ops/src/attention/kernels.rs:683-997,
// re-laid out for CDNA4): a workgroup of 4 wavefronts takes 128 queries of one head, each
// wavefront 32 of them, and sweeps the keys they see in tiles of 64. Per tile:
//   S^T = K Q^T        v_mfma_f32_32x32x16: A = K rows from LDS (16-byte reads along D),
//                      B = this wavefront's queries, held in registers for the whole sweep;
//   online softmax     each lane holds one query's column of S^T, so the row statistics are
//                      per lane plus one exchange with the lane 32 away; exp2 in f32;
//   O^T += V^T P^T     P^T stays in registers as the B operand (the output layout of the first
//                      product, with the key order chosen to match), A = V^T read from a
//                      transposed LDS copy of the V tile (8-byte reads along the keys).
// Scores are masked element by element only on tiles the rows' visibility intervals cut (the
// bottom-right aligned causal/window/packed intervals of dm_common.h, plus key padding).
#include <string>

#include "attention_kernels.h"
#include "mfma.h"

namespace dm {

constexpr int kFwdM = 128;  // queries per workgroup
constexpr int kFwdN = 64;   // keys per tile
// A row-major LDS tile read along its rows by ds_read_b128 (16 lanes on 16 consecutive rows) is
// conflict-free with a row stride of 16 mod 256 bytes; one read transposed by
// ds_read_b64_tr_b16 (a 16-lane group on 4 consecutive rows x 32 bytes, the two groups of a half
// wave side by side) with a stride of 64 mod 256 bytes.
template <int D>
struct Strides {
    static constexpr int ROW = D + 8;   // elements: 272 bytes at D = 128, 144 at D = 64
    static constexpr int TR = D + 32;   // elements: 320 bytes at D = 128, 192 at D = 64
};

template <int D>
struct FwdSlot {
    uint4 k[kFwdN * Strides<D>::ROW / 8];
    uint4 v[kFwdN * Strides<D>::TR / 8];
};

template <int D>
struct FwdSmem {
    FwdSlot<D> slot[2];  // key / value tiles, double-buffered
    int32_t lo[4], hi[4], flo[4], fhi[4];
};

// The per-tile rescale is skipped until a row's maximum grows by more than 2^8 over the one its
// exponentials are taken against: p stays below 256, exact in f32 and bf16 range, and the
// normalisation at the end uses the same reference.
constexpr float kRescaleThreshold = 8.f;

template <int DT, int D, bool PAD>
__global__ __launch_bounds__(256, 2) void attn_fwd_mfma(MaskInfo m, int64_t B, int64_t Hq,
                                                        int64_t Hkv, float scale,
                                                        const uint16_t *__restrict__ q,
                                                        const uint16_t *__restrict__ k,
                                                        const uint16_t *__restrict__ v,
                                                        uint16_t *__restrict__ o,
                                                        float *__restrict__ lse) {
    using Sm = FwdSmem<D>;
    constexpr int KS = Strides<D>::ROW, VS = Strides<D>::TR;
    __shared__ Sm sm;
    constexpr int KSTEPS = D / 16;  // k-steps of S^T over the head dimension
    constexpr int DT32 = D / 32;    // 32-row tiles of O^T
    const int64_t Tq = m.tq, Tk = m.tk;
    const int64_t ntiles = (Tq + kFwdM - 1) / kFwdM;
    const int64_t nwork = ntiles * Hq * B;
    const int64_t work = blockIdx.x;
    if (work >= nwork) return;
    // heads fastest (a key-value group's query heads share K/V in one L2), then tiles from the
    // longest (last) down, then batch
    // the key-value head is the fastest index: consecutive blocks go to consecutive XCDs, so
    // an XCD (with Hkv = 8) holds one key-value head, whose keys and values stay in its L2,
    // and every XCD gets query tiles of every length (the longest first)
    const int64_t kh = work % Hkv;
    const int64_t h = kh * (Hq / Hkv) + (work / Hkv) % (Hq / Hkv);
    const int64_t tile = ntiles - 1 - (work / Hq) % ntiles;
    const int64_t b = work / (Hq * ntiles);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int64_t qi = tile * kFwdM + wave * 32 + col;  // this lane's query row
    const bool qvalid = qi < Tq;

    // visibility interval of this lane's query
    int64_t lo64 = 0, hi64 = 0;
    if (qvalid) row_bounds(m, qi, &lo64, &hi64);
    const int32_t lo = (int32_t)lo64, hi = (int32_t)hi64;
    {
        // workgroup range (union of the rows' intervals) and the keys every row sees; a row
        // that sees nothing forces masking on every tile
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
            sm.lo[wave] = wl;
            sm.hi[wave] = wh;
            sm.flo[wave] = rfl;
            sm.fhi[wave] = rfh;
        }
    }
    __syncthreads();
    const int32_t kv_lo = min(min(sm.lo[0], sm.lo[1]), min(sm.lo[2], sm.lo[3]));
    const int32_t kv_hi = max(max(sm.hi[0], sm.hi[1]), max(sm.hi[2], sm.hi[3]));
    const int32_t full_lo = max(max(sm.flo[0], sm.flo[1]), max(sm.flo[2], sm.flo[3]));
    const int32_t full_hi = min(min(sm.fhi[0], sm.fhi[1]), min(sm.fhi[2], sm.fhi[3]));

    // this wavefront's queries as the B operand: col = query, k = head dimension
    Frag8 qf[KSTEPS];
    {
        const uint16_t *qp = q + ((b * Tq + qi) * Hq + h) * D + half * 8;
#pragma unroll
        for (int s = 0; s < KSTEPS; s++)
            qf[s].u = qvalid ? *(const uint4 *)(qp + s * 16) : make_uint4(0, 0, 0, 0);
    }

    f32x16_t acc[DT32];
#pragma unroll
    for (int t = 0; t < DT32; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[t][i] = 0.f;
    // mc: the reference the exponentials are taken against, max raw score x scale x log2(e);
    // lrow: this lane's partial sum of the exponentials
    float mc = -INFINITY, lrow = 0.f;
    const float c2 = scale * 1.4426950408889634f;

    // staging of one K and one V tile: 16-byte chunks at per-thread byte offsets, loaded through
    // buffer resources whose range ends at the last key (rows past it read as zeros)
    const int32_t kvstride = (int32_t)(Hkv * D);
    const uint32_t kvbytes = (uint32_t)(((Tk - 1) * Hkv + 1) * D * 2);
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(k + (b * Tk * Hkv + kh) * D, kvbytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(v + (b * Tk * Hkv + kh) * D, kvbytes);
    const uint8_t *pad = PAD ? m.pad + b * Tk : nullptr;
    constexpr int CPR = D / 8;                 // chunks per row
    constexpr int NCH = kFwdN * CPR / 256;     // chunks per thread per tensor
    constexpr int RSTEP = 256 / CPR;           // rows between a thread's chunks
    const int crow = tid / CPR, ccol = tid % CPR;
    const uint32_t goff = (uint32_t)(crow * kvstride + ccol * 8) * 2;
    // Tiles go HBM -> registers -> LDS: two register sets, a tile's loads issued two steps
    // before its store (every call issues the same loads; tiles past the range re-read the
    // first), two LDS slots, one barrier per step.
    struct KvStage {
        uint4 k[NCH], v[NCH];
    };
    KvStage st0, st1;
    auto load_tile = [&](KvStage &x, int32_t j0) __attribute__((always_inline)) {
        const uint32_t base = (uint32_t)j0 * (uint32_t)kvstride * 2 + goff;
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            const uint32_t off = base + (uint32_t)(u * RSTEP * kvstride * 2);
            x.k[u] = buf_load16(krs, off);
            x.v[u] = buf_load16(vrs, off);
        }
    };
    auto store_tile = [&](const KvStage &x, FwdSlot<D> &sl) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            sl.k[(crow + u * RSTEP) * (KS / 8) + ccol] = x.k[u];
            sl.v[(crow + u * RSTEP) * (VS / 8) + ccol] = x.v[u];
        }
    };
    auto clampj = [&](int32_t j) { return j < kv_hi ? j : kv_lo; };

    auto one = [&](const int32_t j0, const int sl_cur, KvStage &x) __attribute__((always_inline)) {
        if (j0 + kFwdN < kv_hi) store_tile(x, sm.slot[sl_cur ^ 1]);
        load_tile(x, clampj(j0 + 3 * kFwdN));
        const uint16_t *sk = (const uint16_t *)sm.slot[sl_cur].k;
        const uint16_t *sv = (const uint16_t *)sm.slot[sl_cur].v;

        // S^T for keys [j0, j0 + 64): two 32-key row tiles, their accumulation chains
        // interleaved
        f32x16_t s[2];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) s[t][i] = 0.f;
#pragma unroll
        for (int st = 0; st < KSTEPS; st++)
#pragma unroll
            for (int t = 0; t < 2; t++) {
                Frag8 a;
                a.u = *(const uint4 *)(sk + (t * 32 + col) * KS + half * 8 + st * 16);
                s[t] = mfma32<DT>(a, qf[st], s[t]);
            }
        // mask where the tile is cut
        if (PAD || j0 < full_lo || j0 + kFwdN > full_hi) {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int32_t j = j0 + t * 32 + (i / 4) * 8 + half * 4 + (i % 4);
                    bool vis = (j >= lo) & (j < hi);
                    if constexpr (PAD) vis = vis & (pad[j < Tk ? j : Tk - 1] == 0);
                    s[t][i] = vis ? s[t][i] : -INFINITY;
                }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) tmax = fmaxf(tmax, s[t][i]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float tmc = tmax * c2;
        const bool grow = tmc - mc > kRescaleThreshold;  // false while both are -inf
        if (__any(grow)) {
            const float mnew = grow ? tmc : mc;
            const float alpha = grow ? fast_exp2(mc - mnew) : 1.f;  // 0 from -inf
            mc = mnew;
            lrow *= alpha;
#pragma unroll
            for (int t = 0; t < DT32; t++)
#pragma unroll
                for (int i = 0; i < 16; i++) acc[t][i] *= alpha;
        }
        const float mneg = mc == -INFINITY ? 0.f : -mc;
        // P^T as B fragments: tile t, step u takes the lane's values i in [8u, 8u + 8)
        Frag8 pf[2][2];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                float p[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    p[e] = fast_exp2(fmaf(s[t][8 * u + e], c2, mneg));
                    lrow += p[e];
                }
                pf[t][u].u = make_uint4(pack2<DT>(p[0], p[1]), pack2<DT>(p[2], p[3]),
                                        pack2<DT>(p[4], p[5]), pack2<DT>(p[6], p[7]));
            }
        // O^T += V^T P^T: A = V^T from the row-major V tile by transposed reads, key order
        //   32 t + 16 u + 8 (e / 4) + 4 h + e % 4 in slot e of lane half h of step (t, u);
        // the four output tiles' chains interleaved
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int dt = 0; dt < DT32; dt++) {
                    const Frag8 a = lds_tr_frag(sv, VS, t * 32 + u * 16, dt * 32, lane);
                    acc[dt] = mfma32<DT>(a, pf[t][u], acc[dt]);
                }
        __syncthreads();
    };
    if (kv_lo < kv_hi) {
        load_tile(st0, kv_lo);
        store_tile(st0, sm.slot[0]);
        load_tile(st0, clampj(kv_lo + kFwdN));
        load_tile(st1, clampj(kv_lo + 2 * kFwdN));
    }
    __syncthreads();
    for (int32_t j0 = kv_lo; j0 < kv_hi; j0 += 2 * kFwdN) {
        one(j0, 0, st0);
        if (j0 + kFwdN >= kv_hi) break;
        one(j0 + kFwdN, 1, st1);
    }

    // finish: l over both halves, normalise, write O and lse
    const float ltot = lrow + __shfl_xor(lrow, 32, 64);
    if (!qvalid) return;
    const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
    uint16_t *op = o + ((b * Tq + qi) * Hq + h) * D;
#pragma unroll
    for (int dt = 0; dt < DT32; dt++)
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
            const int d = dt * 32 + g4 * 8 + half * 4;
            uint2 w;
            w.x = pack2<DT>(acc[dt][g4 * 4 + 0] * inv, acc[dt][g4 * 4 + 1] * inv);
            w.y = pack2<DT>(acc[dt][g4 * 4 + 2] * inv, acc[dt][g4 * 4 + 3] * inv);
            *(uint2 *)(op + d) = w;
        }
    if (half == 0)
        lse[(b * Tq + qi) * Hq + h] =
            ltot > 0.f ? (float)((double)mc * 0.6931471805599453 + log((double)ltot)) : -INFINITY;
}

bool mfma_fwd_takes(const dm_attention_desc *d) {
    // a positive scale keeps the maximum of the raw scores the maximum of the scaled ones
    // buffer loads take 32-bit byte offsets within one batch row's keys and values
    return (d->dtype == DM_BF16 || d->dtype == DM_F16) && (d->d == 64 || d->d == 128) &&
           d->tq < (1ll << 30) && d->tk < (1ll << 30) && scale_of(d) > 0.f &&
           d->tk * d->hkv * d->d * 2 < (1ll << 31);
}

int launch_attn_fwd_mfma(const MaskInfo &m, const dm_attention_desc *d, float scale,
                         const void *q, const void *k, const void *v, void *o, float *lse,
                         hipStream_t st) {
    const int64_t ntiles = (d->tq + kFwdM - 1) / kFwdM;
    const int64_t nwork = ntiles * d->hq * d->b;
    const int64_t nblocks = (nwork + 7) / 8 * 8;
    if (nblocks >= (1ll << 31)) return refuse("attention: too many query tiles");
    dim3 grid((unsigned)nblocks), block(256);
    const uint16_t *qq = (const uint16_t *)q, *kk = (const uint16_t *)k, *vv = (const uint16_t *)v;
    uint16_t *oo = (uint16_t *)o;
#define FWD(DT, DD)                                                                            \
    if (m.pad)                                                                                 \
        attn_fwd_mfma<DT, DD, true><<<grid, block, 0, st>>>(m, d->b, d->hq, d->hkv, scale, qq, \
                                                            kk, vv, oo, lse);                 \
    else                                                                                       \
        attn_fwd_mfma<DT, DD, false><<<grid, block, 0, st>>>(m, d->b, d->hq, d->hkv, scale,   \
                                                             qq, kk, vv, oo, lse)
    {
        KernelTimer timer(DM_KERNEL_ATTN_FWD, st);
        if (d->dtype == DM_BF16) {
            if (d->d == 64) { FWD(DM_BF16, 64); } else { FWD(DM_BF16, 128); }
        } else {
            if (d->d == 64) { FWD(DM_F16, 64); } else { FWD(DM_F16, 128); }
        }
    }
#undef FWD
    probe_add(DM_PROBE_ATTN_FWD_MFMA);
    DM_LAUNCH_CHECK("attention: MFMA forward launch");
    return DM_OK;
}

}  // namespace dm
