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

template <int D>
struct FwdSmem {
    static constexpr int KS = D + 8;   // K row stride (elements): 16-byte pad against conflicts
    static constexpr int VS = kFwdN + 4;  // V^T row stride: 136 bytes, conflict-free 8-byte reads
    uint16_t k[kFwdN * KS];
    uint16_t vt[D * VS];
    int32_t lo[4], hi[4], flo[4], fhi[4];
};

template <int DT, int D>
__global__ __launch_bounds__(256, 2) void attn_fwd_mfma(MaskInfo m, int64_t B, int64_t Hq,
                                                        int64_t Hkv, float scale,
                                                        const uint16_t *__restrict__ q,
                                                        const uint16_t *__restrict__ k,
                                                        const uint16_t *__restrict__ v,
                                                        uint16_t *__restrict__ o,
                                                        float *__restrict__ lse) {
    using Sm = FwdSmem<D>;
    __shared__ Sm sm;
    constexpr int KSTEPS = D / 16;  // k-steps of S^T over the head dimension
    constexpr int DT32 = D / 32;    // 32-row tiles of O^T
    const int64_t Tq = m.tq, Tk = m.tk;
    const int64_t ntiles = (Tq + kFwdM - 1) / kFwdM;
    const int64_t nwork = ntiles * Hq * B;
    const int64_t work = xcd_remap(blockIdx.x, gridDim.x);
    if (work >= nwork) return;
    // heads fastest (a key-value group's query heads share K/V in one L2), then tiles from the
    // longest (last) down, then batch
    const int64_t h = work % Hq;
    const int64_t tile = ntiles - 1 - (work / Hq) % ntiles;
    const int64_t b = work / (Hq * ntiles);
    const int64_t kh = h / (Hq / Hkv);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int64_t m0 = tile * kFwdM;
    const int64_t qi = m0 + wave * 32 + col;  // this lane's query row
    const bool qvalid = qi < Tq;

    // visibility interval of this lane's query
    int64_t lo = 0, hi = 0;
    if (qvalid) row_bounds(m, qi, &lo, &hi);
    // workgroup range: union of the rows' intervals; the keys every row sees
    {
        int32_t wl = lo < hi ? (int32_t)lo : INT32_MAX, wh = lo < hi ? (int32_t)hi : INT32_MIN;
        // rows that see nothing force masking on every tile
        int32_t fl = lo < hi ? (int32_t)lo : INT32_MAX, fh = lo < hi ? (int32_t)hi : INT32_MIN;
        int32_t rfl = (qvalid && lo < hi) ? (int32_t)lo : (qvalid ? INT32_MAX : INT32_MIN);
        int32_t rfh = (qvalid && lo < hi) ? (int32_t)hi : (qvalid ? INT32_MIN : INT32_MAX);
        (void)fl;
        (void)fh;
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
    const int64_t qstride = Hq * D;  // elements between consecutive query rows
    Frag8 qf[KSTEPS];
    {
        const uint16_t *qp = q + ((b * Tq + qi) * Hq + h) * D + half * 8;
#pragma unroll
        for (int s = 0; s < KSTEPS; s++)
            qf[s].u = qvalid ? *(const uint4 *)(qp + s * 16) : make_uint4(0, 0, 0, 0);
    }
    (void)qstride;

    f32x16_t acc[DT32];
#pragma unroll
    for (int t = 0; t < DT32; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[t][i] = 0.f;
    float mrow = -INFINITY, lrow = 0.f;  // running max of the raw scores, this lane's partial sum
    const float qk_scale = scale * 1.4426950408889634f;

    const int64_t kvstride = Hkv * D;  // elements between consecutive key rows
    const uint16_t *kbase = k + (b * Tk * Hkv + kh) * D;
    const uint16_t *vbase = v + (b * Tk * Hkv + kh) * D;
    const uint8_t *pad = m.pad ? m.pad + b * Tk : nullptr;

    // global -> register staging of one K tile (16-byte chunks) and one V tile (4x4 blocks)
    constexpr int KCH = kFwdN * D / 8 / 256;       // K chunks per thread
    constexpr int VBL = kFwdN * D / 16 / 256;      // V 4x4 blocks per thread
    uint4 kreg[KCH];
    uint2 vreg[VBL][4];
    auto load_tile = [&](int64_t j0) {
#pragma unroll
        for (int u = 0; u < KCH; u++) {
            const int c = tid + 256 * u;
            const int r = c / (D / 8), c8 = c % (D / 8);
            const int64_t j = j0 + r;
            kreg[u] = j < Tk ? *(const uint4 *)(kbase + j * kvstride + c8 * 8)
                             : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < VBL; u++) {
            const int c = tid + 256 * u;
            const int dq = c % (D / 4), kq = c / (D / 4);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t j = j0 + kq * 4 + r;
                vreg[u][r] = j < Tk ? *(const uint2 *)(vbase + j * kvstride + dq * 4)
                                    : make_uint2(0, 0);
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int u = 0; u < KCH; u++) {
            const int c = tid + 256 * u;
            const int r = c / (D / 8), c8 = c % (D / 8);
            *(uint4 *)(sm.k + r * Sm::KS + c8 * 8) = kreg[u];
        }
#pragma unroll
        for (int u = 0; u < VBL; u++) {
            const int c = tid + 256 * u;
            const int dq = c % (D / 4), kq = c / (D / 4);
            const uint2 *x = vreg[u];
            // 4 keys x 4 dims -> 4 dims x 4 keys
            uint2 t0, t1, t2, t3;
            t0.x = (x[0].x & 0xffffu) | (x[1].x << 16);
            t0.y = (x[2].x & 0xffffu) | (x[3].x << 16);
            t1.x = (x[0].x >> 16) | (x[1].x & 0xffff0000u);
            t1.y = (x[2].x >> 16) | (x[3].x & 0xffff0000u);
            t2.x = (x[0].y & 0xffffu) | (x[1].y << 16);
            t2.y = (x[2].y & 0xffffu) | (x[3].y << 16);
            t3.x = (x[0].y >> 16) | (x[1].y & 0xffff0000u);
            t3.y = (x[2].y >> 16) | (x[3].y & 0xffff0000u);
            uint16_t *dst = sm.vt + (dq * 4) * Sm::VS + kq * 4;
            *(uint2 *)(dst) = t0;
            *(uint2 *)(dst + Sm::VS) = t1;
            *(uint2 *)(dst + 2 * Sm::VS) = t2;
            *(uint2 *)(dst + 3 * Sm::VS) = t3;
        }
    };

    if (kv_lo < kv_hi) load_tile(kv_lo);
    for (int64_t j0 = kv_lo; j0 < kv_hi; j0 += kFwdN) {
        __syncthreads();
        store_tile();
        __syncthreads();
        if (j0 + kFwdN < kv_hi) load_tile(j0 + kFwdN);

        // S^T for keys [j0, j0 + 64): two 32-key row tiles
        f32x16_t s[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int i = 0; i < 16; i++) s[t][i] = 0.f;
            const uint16_t *kr = sm.k + (t * 32 + col) * Sm::KS + half * 8;
#pragma unroll
            for (int st = 0; st < KSTEPS; st++) {
                Frag8 a;
                a.u = *(const uint4 *)(kr + st * 16);
                s[t] = mfma32<DT>(a, qf[st], s[t]);
            }
        }
        // mask where the tile is cut; the row statistics are kept on the raw scores, so that
        // p = exp2((s - m) * scale * log2(e)) rounds once after an exact subtraction
        const bool masked = pad || j0 < full_lo || j0 + kFwdN > full_hi;
        float tmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                float x = s[t][i];
                if (masked) {
                    const int64_t j = j0 + t * 32 + (i / 4) * 8 + half * 4 + (i % 4);
                    const bool vis = j >= lo && j < hi && (!pad || !pad[j]);
                    x = vis ? x : -INFINITY;
                }
                s[t][i] = x;
                tmax = fmaxf(tmax, x);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float mnew = fmaxf(mrow, tmax);
        const float mbase = mnew == -INFINITY ? 0.f : mnew;
        const float alpha = exp2f((mrow - mbase) * qk_scale);
        mrow = mnew;
        lrow *= alpha;
#pragma unroll
        for (int t = 0; t < DT32; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[t][i] *= alpha;
        // P^T as B fragments: tile t, step u takes the lane's values i in [8u, 8u + 8)
        Frag8 pf[2][2];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                float p[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    p[e] = exp2f((s[t][8 * u + e] - mbase) * qk_scale);
                    lrow += p[e];
                }
                pf[t][u].u = make_uint4(pack2<DT>(p[0], p[1]), pack2<DT>(p[2], p[3]),
                                        pack2<DT>(p[4], p[5]), pack2<DT>(p[6], p[7]));
            }
        // O^T += V^T P^T: key order of slot e of lane half h in step (t, u):
        //   32 t + 16 u + 8 (e / 4) + 4 h + e % 4
#pragma unroll
        for (int dt = 0; dt < DT32; dt++) {
            const uint16_t *vr = sm.vt + (dt * 32 + col) * Sm::VS + half * 4;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const uint16_t *p0 = vr + t * 32 + u * 16;
                    const uint2 lo4 = *(const uint2 *)(p0);
                    const uint2 hi4 = *(const uint2 *)(p0 + 8);
                    Frag8 a;
                    a.u = make_uint4(lo4.x, lo4.y, hi4.x, hi4.y);
                    acc[dt] = mfma32<DT>(a, pf[t][u], acc[dt]);
                }
        }
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
            ltot > 0.f ? (float)((double)mrow * (double)scale + log((double)ltot)) : -INFINITY;
}

bool mfma_fwd_takes(const dm_attention_desc *d) {
    // a positive scale keeps the maximum of the raw scores the maximum of the scaled ones
    return (d->dtype == DM_BF16 || d->dtype == DM_F16) && (d->d == 64 || d->d == 128) &&
           d->tq < (1ll << 30) && d->tk < (1ll << 30) && scale_of(d) > 0.f;
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
#define FWD(DT, DD) \
    attn_fwd_mfma<DT, DD><<<grid, block, 0, st>>>(m, d->b, d->hq, d->hkv, scale, qq, kk, vv, oo, lse)
    if (d->dtype == DM_BF16) {
        if (d->d == 64) FWD(DM_BF16, 64); else FWD(DM_BF16, 128);
    } else {
        if (d->d == 64) FWD(DM_F16, 64); else FWD(DM_F16, 128);
    }
#undef FWD
    probe_add(DM_PROBE_ATTN_FWD_MFMA);
    DM_LAUNCH_CHECK("attention: MFMA forward launch");
    return DM_OK;
}

}  // namespace dm
