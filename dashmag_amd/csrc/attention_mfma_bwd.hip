// MFMA attention backward for gfx950 (bf16/f16, head width 64 or 128), deterministic: the
// query gradient is summed over the key tiles in a fixed order by its own sweep, as the
// reference's default does (crates/dash-ops/src/attention/kernels.rs:999-2058; the contract's
// `deterministic`, crates/dash-contract/src/attention.rs:100-105).
//
//   bwd_prep   per query row: delta = rowsum(dO o O), lse in log2 units (+inf for a row that
//              sees no key, so its probabilities are 0), the row's visibility interval; per tile
//              of 64 rows the union of the intervals and the keys every row sees.
//   bwd_dkdv   per (tile of 128 keys, key-value head): sweeps the query heads of the group and
//              the 64-query tiles that see the keys. The keys and values stay in registers as the
//              B operands of S = Q K^T and dP = dO V^T (v_mfma_f32_32x32x16); P and dS go from the
//              products' output layout straight into the A operands of dV += P^T dO and
//              dK += dS^T Q, whose B operands come from transposed LDS copies of the tile.
//   bwd_dq     per (tile of 128 queries, query head): sweeps the key tiles as the forward does,
//              recomputing S^T and dP^T, dQ^T += K^T dS^T.
#include <string>

#include "attention_kernels.h"
#include "mfma.h"

namespace dm {

constexpr int kRowTile = 64;   // rows per tile of the prep's tile ranges
constexpr int kKvBlock = 128;  // keys per dK/dV workgroup (32 per wavefront)
constexpr int kQTile = 64;     // queries per step of the dK/dV sweep
constexpr int kDqM = 128;      // queries per dQ workgroup
constexpr int kDqN = 64;       // keys per step of the dQ sweep

struct BwdWs {
    float *lse2;      // [B, Tq, Hq]
    int32_t *rlo;     // [B, Tq]
    int32_t *rhi;     // [B, Tq]
    int32_t *trange;  // [B, ntiles, 4]: union lo, union hi, full lo, full hi
};

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
    x.rlo = (int32_t *)take(qrows * 4);
    x.rhi = (int32_t *)take(qrows * 4);
    x.trange = (int32_t *)take(d->b * ntiles * 4 * 4);
    if (w) *w = x;
    return off;
}

// ------------------------------------------------------------------------------------------
// Prep
// ------------------------------------------------------------------------------------------

template <int DT, int D>
__global__ __launch_bounds__(256) void bwd_prep(MaskInfo m, int64_t B, int64_t Hq,
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
    constexpr int CH = D / 8;  // 16-byte chunks per head row
    for (int64_t h = lane / CH; h < Hq; h += 64 / CH) {
        const int c = lane % CH;
        const int64_t base = (row * Hq + h) * D + c * 8;
        const uint4 a = *(const uint4 *)(o + base), g = *(const uint4 *)(d_o + base);
        float s = unpack_lo<DT>(a.x) * unpack_lo<DT>(g.x) + unpack_hi<DT>(a.x) * unpack_hi<DT>(g.x) +
                  unpack_lo<DT>(a.y) * unpack_lo<DT>(g.y) + unpack_hi<DT>(a.y) * unpack_hi<DT>(g.y) +
                  unpack_lo<DT>(a.z) * unpack_lo<DT>(g.z) + unpack_hi<DT>(a.z) * unpack_hi<DT>(g.z) +
                  unpack_lo<DT>(a.w) * unpack_lo<DT>(g.w) + unpack_hi<DT>(a.w) * unpack_hi<DT>(g.w);
#pragma unroll
        for (int off = CH / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
        if (c == 0) {
            delta[row * Hq + h] = s;
            const float l = lse[row * Hq + h];
            w.lse2[row * Hq + h] = l == -INFINITY ? INFINITY : l * 1.4426950408889634f;
        }
    }
    (void)b;
}

// Per tile of 64 rows: [union lo, union hi) of the rows' intervals, and [full lo, full hi), the
// keys every row of the tile sees (empty when a row of the tile sees nothing).
__global__ __launch_bounds__(64) void bwd_tiles(int64_t B, int64_t Tq, BwdWs w) {
    const int64_t ntiles = (Tq + kRowTile - 1) / kRowTile;
    const int64_t t = blockIdx.x;
    if (t >= B * ntiles) return;
    const int64_t b = t / ntiles, tile = t % ntiles;
    const int64_t i = tile * kRowTile + threadIdx.x;
    int32_t ul = INT32_MAX, uh = INT32_MIN, fl = INT32_MIN, fh = INT32_MAX;
    if (i < Tq) {
        const int32_t lo = w.rlo[b * Tq + i], hi = w.rhi[b * Tq + i];
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

// 4 rows x 4 columns of 16-bit values (4 uint2, one per row) -> 4 columns x 4 rows.
__device__ __forceinline__ void transpose4(const uint2 *x, uint2 *t) {
    t[0].x = (x[0].x & 0xffffu) | (x[1].x << 16);
    t[0].y = (x[2].x & 0xffffu) | (x[3].x << 16);
    t[1].x = (x[0].x >> 16) | (x[1].x & 0xffff0000u);
    t[1].y = (x[2].x >> 16) | (x[3].x & 0xffff0000u);
    t[2].x = (x[0].y & 0xffffu) | (x[1].y << 16);
    t[2].y = (x[2].y & 0xffffu) | (x[3].y << 16);
    t[3].x = (x[0].y >> 16) | (x[1].y & 0xffff0000u);
    t[3].y = (x[2].y >> 16) | (x[3].y & 0xffff0000u);
}

// ------------------------------------------------------------------------------------------
// dK, dV
// ------------------------------------------------------------------------------------------

template <int D>
struct DkdvSmem {
    static constexpr int RS = D + 8;       // row-major stride (elements)
    static constexpr int TS = kQTile + 4;  // transposed stride: 136 bytes
    uint16_t q[kQTile * RS];
    uint16_t qt[D * TS];
    uint16_t g[kQTile * RS];
    uint16_t gt[D * TS];
    float lse2[kQTile], delta[kQTile];
    int32_t rlo[kQTile], rhi[kQTile];
};

template <int DT, int D>
__global__ __launch_bounds__(256, 1) void bwd_dkdv(MaskInfo m, int64_t B, int64_t Hq,
                                                   int64_t Hkv, float scale,
                                                   const uint16_t *__restrict__ q,
                                                   const uint16_t *__restrict__ k,
                                                   const uint16_t *__restrict__ v,
                                                   const uint16_t *__restrict__ d_o,
                                                   const float *__restrict__ delta,
                                                   BwdWs w, uint16_t *__restrict__ dk,
                                                   uint16_t *__restrict__ dv) {
    using Sm = DkdvSmem<D>;
    __shared__ Sm sm;
    constexpr int KSTEPS = D / 16, DT32 = D / 32;
    const int64_t Tq = m.tq, Tk = m.tk;
    const int64_t nkb = (Tk + kKvBlock - 1) / kKvBlock;
    const int64_t nwork = nkb * Hkv * B;
    const int64_t work = xcd_remap(blockIdx.x, gridDim.x);
    if (work >= nwork) return;
    const int64_t kh = work % Hkv, kb = (work / Hkv) % nkb, b = work / (Hkv * nkb);
    const int64_t group = Hq / Hkv;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int64_t j0 = kb * kKvBlock;
    const int64_t key = j0 + wave * 32 + col;  // this lane's key
    const bool kvalid = key < Tk;
    const bool kpad = m.pad && kvalid && m.pad[b * Tk + key];
    const int64_t kvstride = Hkv * D, qstride = Hq * D;
    const float c2 = scale * 1.4426950408889634f;

    // K and V of this lane's key as B operands (col = key, k = head dimension)
    Frag8 kf[KSTEPS], vf[KSTEPS];
    {
        const uint16_t *kp = k + ((b * Tk + key) * Hkv + kh) * D + half * 8;
        const uint16_t *vp = v + ((b * Tk + key) * Hkv + kh) * D + half * 8;
#pragma unroll
        for (int s = 0; s < KSTEPS; s++) {
            kf[s].u = kvalid ? *(const uint4 *)(kp + s * 16) : make_uint4(0, 0, 0, 0);
            vf[s].u = kvalid ? *(const uint4 *)(vp + s * 16) : make_uint4(0, 0, 0, 0);
        }
    }
    f32x16_t dka[DT32], dva[DT32];
#pragma unroll
    for (int t = 0; t < DT32; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) dka[t][i] = dva[t][i] = 0.f;

    const int64_t ntiles = (Tq + kQTile - 1) / kQTile;
    const int32_t *tr = w.trange + b * ntiles * 4;
    const int64_t j1 = j0 + kKvBlock < Tk ? j0 + kKvBlock : Tk;
    auto sees = [&](int64_t t) -> bool { return tr[t * 4] < j1 && tr[t * 4 + 1] > j0; };

    // staging: Q and dO tiles as 4x4 blocks (row-major and transposed copies come from them)
    constexpr int NB = kQTile * D / 16 / 256;  // 4x4 blocks per thread per tensor
    uint2 qreg[NB][4], greg[NB][4];
    auto load = [&](int64_t h, int64_t t) {
        const int64_t i0 = t * kQTile;
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const int c = tid + 256 * u;
            const int dq = c % (D / 4), rq = c / (D / 4);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t i = i0 + rq * 4 + r;
                const bool ok = i < Tq;
                const int64_t off = ((b * Tq + i) * Hq + h) * D + dq * 4;
                qreg[u][r] = ok ? *(const uint2 *)(q + off) : make_uint2(0, 0);
                greg[u][r] = ok ? *(const uint2 *)(d_o + off) : make_uint2(0, 0);
            }
        }
    };
    float st_lse = 0.f, st_delta = 0.f;
    int32_t st_lo = 0, st_hi = 0;
    auto load_rows = [&](int64_t h, int64_t t) {
        if (tid < kQTile) {
            const int64_t i = t * kQTile + tid;
            const bool ok = i < Tq;
            st_lse = ok ? w.lse2[(b * Tq + i) * Hq + h] : INFINITY;
            st_delta = ok ? delta[(b * Tq + i) * Hq + h] : 0.f;
            st_lo = ok ? w.rlo[b * Tq + i] : 0;
            st_hi = ok ? w.rhi[b * Tq + i] : 0;
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const int c = tid + 256 * u;
            const int dq = c % (D / 4), rq = c / (D / 4);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                *(uint2 *)(sm.q + (rq * 4 + r) * Sm::RS + dq * 4) = qreg[u][r];
                *(uint2 *)(sm.g + (rq * 4 + r) * Sm::RS + dq * 4) = greg[u][r];
            }
            uint2 t4[4];
            transpose4(qreg[u], t4);
#pragma unroll
            for (int e = 0; e < 4; e++) *(uint2 *)(sm.qt + (dq * 4 + e) * Sm::TS + rq * 4) = t4[e];
            transpose4(greg[u], t4);
#pragma unroll
            for (int e = 0; e < 4; e++) *(uint2 *)(sm.gt + (dq * 4 + e) * Sm::TS + rq * 4) = t4[e];
        }
        if (tid < kQTile) {
            sm.lse2[tid] = st_lse;
            sm.delta[tid] = st_delta;
            sm.rlo[tid] = st_lo;
            sm.rhi[tid] = st_hi;
        }
    };

    // the (head, tile) steps: the group's query heads, each over the tiles that see the keys
    int64_t hh = kh * group, tt = 0;
    auto advance = [&](int64_t &h, int64_t &t) {
        // from (h, t) to the next step that sees the keys, or h = end
        while (h < (kh + 1) * group) {
            while (t < ntiles && !sees(t)) t++;
            if (t < ntiles) return;
            h++;
            t = 0;
        }
    };
    const bool any_key = j0 < Tk;
    if (any_key) advance(hh, tt);
    if (any_key && hh < (kh + 1) * group) {
        load(hh, tt);
        load_rows(hh, tt);
    }
    while (any_key && hh < (kh + 1) * group) {
        const int64_t h = hh, t = tt;
        __syncthreads();
        store();
        __syncthreads();
        // next step's loads, in flight during this step's products
        tt++;
        advance(hh, tt);
        if (hh < (kh + 1) * group) {
            load(hh, tt);
            load_rows(hh, tt);
        }
        const int32_t *r = tr + t * 4;
        const bool masked = m.pad != nullptr || r[2] > j0 || r[3] < j0 + kKvBlock;
#pragma unroll
        for (int qs = 0; qs < kQTile / 32; qs++) {
            // S and dP for 32 queries x this wavefront's 32 keys
            f32x16_t s, dp;
#pragma unroll
            for (int i = 0; i < 16; i++) s[i] = dp[i] = 0.f;
            const uint16_t *qa = sm.q + (qs * 32 + col) * Sm::RS + half * 8;
            const uint16_t *ga = sm.g + (qs * 32 + col) * Sm::RS + half * 8;
#pragma unroll
            for (int st = 0; st < KSTEPS; st++) {
                Frag8 a;
                a.u = *(const uint4 *)(qa + st * 16);
                s = mfma32<DT>(a, kf[st], s);
                a.u = *(const uint4 *)(ga + st * 16);
                dp = mfma32<DT>(a, vf[st], dp);
            }
            // P = exp2(S c - lse2), dS = P (dP - delta), element (query row, this lane's key)
            Frag8 pf[2], df[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                float p[8], ds[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int i = 8 * u + e;
                    const int qr = qs * 32 + (i / 4) * 8 + half * 4 + (i % 4);
                    float x = exp2f(s[i] * c2 - sm.lse2[qr]);
                    if (masked) {
                        const bool vis = key >= sm.rlo[qr] && key < sm.rhi[qr] && !kpad;
                        x = vis ? x : 0.f;
                    }
                    p[e] = x;
                    ds[e] = x * (dp[i] - sm.delta[qr]);
                }
                pf[u].u = make_uint4(pack2<DT>(p[0], p[1]), pack2<DT>(p[2], p[3]),
                                     pack2<DT>(p[4], p[5]), pack2<DT>(p[6], p[7]));
                df[u].u = make_uint4(pack2<DT>(ds[0], ds[1]), pack2<DT>(ds[2], ds[3]),
                                     pack2<DT>(ds[4], ds[5]), pack2<DT>(ds[6], ds[7]));
            }
            // dV += P^T dO, dK += dS^T Q: A = (row key, k = query), B = (k = query, col = d)
            // from the transposed copies; slot e of lane half h in step u is query
            //   32 qs + 16 u + 8 (e / 4) + 4 h + e % 4
#pragma unroll
            for (int dt = 0; dt < DT32; dt++) {
                const uint16_t *gp = sm.gt + (dt * 32 + col) * Sm::TS + qs * 32 + half * 4;
                const uint16_t *qp = sm.qt + (dt * 32 + col) * Sm::TS + qs * 32 + half * 4;
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    Frag8 bg, bq;
                    const uint2 g0 = *(const uint2 *)(gp + u * 16), g1 = *(const uint2 *)(gp + u * 16 + 8);
                    const uint2 q0 = *(const uint2 *)(qp + u * 16), q1 = *(const uint2 *)(qp + u * 16 + 8);
                    bg.u = make_uint4(g0.x, g0.y, g1.x, g1.y);
                    bq.u = make_uint4(q0.x, q0.y, q1.x, q1.y);
                    dva[dt] = mfma32<DT>(pf[u], bg, dva[dt]);
                    dka[dt] = mfma32<DT>(df[u], bq, dka[dt]);
                }
            }
        }
        (void)h;
    }
    // write dK (scaled), dV: lane holds column d = 32 dt + col, rows = keys of this wavefront
    //   32 w + 8 (i / 4) + 4 h + i % 4
#pragma unroll
    for (int dt = 0; dt < DT32; dt++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int64_t j = j0 + wave * 32 + (i / 4) * 8 + half * 4 + (i % 4);
            if (j >= Tk) continue;
            const int64_t off = ((b * Tk + j) * Hkv + kh) * D + dt * 32 + col;
            const float kv = dka[dt][i] * scale, vv = dva[dt][i];
            if constexpr (DT == DM_BF16) {
                dk[off] = f32_to_bf16(kv);
                dv[off] = f32_to_bf16(vv);
            } else {
                _Float16 a = (_Float16)kv, c = (_Float16)vv;
                dk[off] = *(uint16_t *)&a;
                dv[off] = *(uint16_t *)&c;
            }
        }
    (void)kvstride;
    (void)qstride;
}

// ------------------------------------------------------------------------------------------
// dQ
// ------------------------------------------------------------------------------------------

template <int D>
struct DqSmem {
    static constexpr int RS = D + 8;
    static constexpr int TS = kDqN + 4;
    uint16_t k[kDqN * RS];
    uint16_t v[kDqN * RS];
    uint16_t kt[D * TS];
    int32_t lo[4], hi[4], flo[4], fhi[4];
};

template <int DT, int D>
__global__ __launch_bounds__(256, 1) void bwd_dq(MaskInfo m, int64_t B, int64_t Hq, int64_t Hkv,
                                                 float scale, const uint16_t *__restrict__ q,
                                                 const uint16_t *__restrict__ k,
                                                 const uint16_t *__restrict__ v,
                                                 const uint16_t *__restrict__ d_o,
                                                 const float *__restrict__ delta, BwdWs w,
                                                 uint16_t *__restrict__ dq) {
    using Sm = DqSmem<D>;
    __shared__ Sm sm;
    constexpr int KSTEPS = D / 16, DT32 = D / 32;
    const int64_t Tq = m.tq, Tk = m.tk;
    const int64_t ntiles = (Tq + kDqM - 1) / kDqM;
    const int64_t nwork = ntiles * Hq * B;
    const int64_t work = xcd_remap(blockIdx.x, gridDim.x);
    if (work >= nwork) return;
    const int64_t h = work % Hq;
    const int64_t tile = ntiles - 1 - (work / Hq) % ntiles;
    const int64_t b = work / (Hq * ntiles);
    const int64_t kh = h / (Hq / Hkv);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int64_t qi = tile * kDqM + wave * 32 + col;
    const bool qvalid = qi < Tq;
    int64_t lo = 0, hi = 0;
    float lse2 = INFINITY, dl = 0.f;
    if (qvalid) {
        lo = w.rlo[b * Tq + qi];
        hi = w.rhi[b * Tq + qi];
        lse2 = w.lse2[(b * Tq + qi) * Hq + h];
        dl = delta[(b * Tq + qi) * Hq + h];
    }
    if (lse2 == INFINITY) hi = lo;  // a query that sees no key: dq = 0
    {
        int32_t wl = lo < hi ? (int32_t)lo : INT32_MAX, wh = lo < hi ? (int32_t)hi : INT32_MIN;
        int32_t rfl = (qvalid && lo < hi) ? (int32_t)lo : (qvalid ? INT32_MAX : INT32_MIN);
        int32_t rfh = (qvalid && lo < hi) ? (int32_t)hi : (qvalid ? INT32_MIN : INT32_MAX);
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

    Frag8 qf[KSTEPS], gf[KSTEPS];
    {
        const int64_t off = ((b * Tq + qi) * Hq + h) * D + half * 8;
#pragma unroll
        for (int s = 0; s < KSTEPS; s++) {
            qf[s].u = qvalid ? *(const uint4 *)(q + off + s * 16) : make_uint4(0, 0, 0, 0);
            gf[s].u = qvalid ? *(const uint4 *)(d_o + off + s * 16) : make_uint4(0, 0, 0, 0);
        }
    }
    f32x16_t acc[DT32];
#pragma unroll
    for (int t = 0; t < DT32; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[t][i] = 0.f;
    const float c2 = scale * 1.4426950408889634f;
    const int64_t kvstride = Hkv * D;
    const uint16_t *kbase = k + (b * Tk * Hkv + kh) * D;
    const uint16_t *vbase = v + (b * Tk * Hkv + kh) * D;
    const uint8_t *pad = m.pad ? m.pad + b * Tk : nullptr;

    constexpr int NB = kDqN * D / 16 / 256;
    uint2 kreg[NB][4], vreg[NB][4];
    auto load_tile = [&](int64_t j0) {
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const int c = tid + 256 * u;
            const int dq4 = c % (D / 4), kq = c / (D / 4);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t j = j0 + kq * 4 + r;
                const bool ok = j < Tk;
                kreg[u][r] = ok ? *(const uint2 *)(kbase + j * kvstride + dq4 * 4) : make_uint2(0, 0);
                vreg[u][r] = ok ? *(const uint2 *)(vbase + j * kvstride + dq4 * 4) : make_uint2(0, 0);
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const int c = tid + 256 * u;
            const int dq4 = c % (D / 4), kq = c / (D / 4);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                *(uint2 *)(sm.k + (kq * 4 + r) * Sm::RS + dq4 * 4) = kreg[u][r];
                *(uint2 *)(sm.v + (kq * 4 + r) * Sm::RS + dq4 * 4) = vreg[u][r];
            }
            uint2 t4[4];
            transpose4(kreg[u], t4);
#pragma unroll
            for (int e = 0; e < 4; e++) *(uint2 *)(sm.kt + (dq4 * 4 + e) * Sm::TS + kq * 4) = t4[e];
        }
    };

    if (kv_lo < kv_hi) load_tile(kv_lo);
    for (int64_t j0 = kv_lo; j0 < kv_hi; j0 += kDqN) {
        __syncthreads();
        store_tile();
        __syncthreads();
        if (j0 + kDqN < kv_hi) load_tile(j0 + kDqN);
        const bool masked = pad || j0 < full_lo || j0 + kDqN > full_hi;
        Frag8 df[2][2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            f32x16_t s, dp;
#pragma unroll
            for (int i = 0; i < 16; i++) s[i] = dp[i] = 0.f;
            const uint16_t *ka = sm.k + (t * 32 + col) * Sm::RS + half * 8;
            const uint16_t *va = sm.v + (t * 32 + col) * Sm::RS + half * 8;
#pragma unroll
            for (int st = 0; st < KSTEPS; st++) {
                Frag8 a;
                a.u = *(const uint4 *)(ka + st * 16);
                s = mfma32<DT>(a, qf[st], s);
                a.u = *(const uint4 *)(va + st * 16);
                dp = mfma32<DT>(a, gf[st], dp);
            }
#pragma unroll
            for (int u = 0; u < 2; u++) {
                float ds[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int i = 8 * u + e;
                    float p = exp2f(s[i] * c2 - lse2);
                    if (masked) {
                        const int64_t j = j0 + t * 32 + (i / 4) * 8 + half * 4 + (i % 4);
                        const bool vis = j >= lo && j < hi && (!pad || !pad[j]);
                        p = vis ? p : 0.f;
                    }
                    ds[e] = p * (dp[i] - dl);
                }
                df[t][u].u = make_uint4(pack2<DT>(ds[0], ds[1]), pack2<DT>(ds[2], ds[3]),
                                        pack2<DT>(ds[4], ds[5]), pack2<DT>(ds[6], ds[7]));
            }
        }
        // dQ^T += K^T dS^T
#pragma unroll
        for (int dt = 0; dt < DT32; dt++) {
            const uint16_t *kr = sm.kt + (dt * 32 + col) * Sm::TS + half * 4;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const uint16_t *p0 = kr + t * 32 + u * 16;
                    const uint2 lo4 = *(const uint2 *)(p0), hi4 = *(const uint2 *)(p0 + 8);
                    Frag8 a;
                    a.u = make_uint4(lo4.x, lo4.y, hi4.x, hi4.y);
                    acc[dt] = mfma32<DT>(a, df[t][u], acc[dt]);
                }
        }
    }
    if (!qvalid) return;
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

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------

bool mfma_bwd_takes(const dm_attention_desc *d) {
    return (d->dtype == DM_BF16 || d->dtype == DM_F16) && (d->d == 64 || d->d == 128) &&
           d->tq < (1ll << 30) && d->tk < (1ll << 30) && scale_of(d) > 0.f;
}

size_t mfma_bwd_workspace(const dm_attention_desc *d) {
    return mfma_bwd_takes(d) ? bwd_layout(d, nullptr, nullptr) : 0;
}

int launch_attn_bwd_mfma(const MaskInfo &m, const dm_attention_desc *d, float scale,
                         const void *q, const void *k, const void *v, const void *o,
                         const float *lse, const void *d_o, void *dq, void *dk, void *dv,
                         float *delta, void *workspace, hipStream_t st) {
    BwdWs w;
    bwd_layout(d, (char *)workspace, &w);
    const int64_t qrows = d->b * d->tq;
    const int64_t ntiles64 = (d->tq + kRowTile - 1) / kRowTile;
    const int64_t nkb = (d->tk + kKvBlock - 1) / kKvBlock;
    const int64_t nq = (d->tq + kDqM - 1) / kDqM;
    const int64_t nb_kv = (nkb * d->hkv * d->b + 7) / 8 * 8;
    const int64_t nb_q = (nq * d->hq * d->b + 7) / 8 * 8;
    if (nb_kv >= (1ll << 31) || nb_q >= (1ll << 31)) return refuse("attention_backward: too large");
    const uint16_t *qq = (const uint16_t *)q, *kk = (const uint16_t *)k, *vv = (const uint16_t *)v;
    const uint16_t *oo = (const uint16_t *)o, *gg = (const uint16_t *)d_o;
#define BWD(DT, DD)                                                                            \
    bwd_prep<DT, DD><<<(unsigned)((qrows + 3) / 4), 256, 0, st>>>(m, d->b, d->hq, oo, gg, lse, \
                                                                   delta, w);                  \
    bwd_tiles<<<(unsigned)(d->b * ntiles64), 64, 0, st>>>(d->b, d->tq, w);                     \
    bwd_dkdv<DT, DD><<<(unsigned)nb_kv, 256, 0, st>>>(m, d->b, d->hq, d->hkv, scale, qq, kk,   \
                                                      vv, gg, delta, w, (uint16_t *)dk,        \
                                                      (uint16_t *)dv);                         \
    bwd_dq<DT, DD><<<(unsigned)nb_q, 256, 0, st>>>(m, d->b, d->hq, d->hkv, scale, qq, kk, vv,  \
                                                   gg, delta, w, (uint16_t *)dq)
    if (d->dtype == DM_BF16) {
        if (d->d == 64) { BWD(DM_BF16, 64); } else { BWD(DM_BF16, 128); }
    } else {
        if (d->d == 64) { BWD(DM_F16, 64); } else { BWD(DM_F16, 128); }
    }
#undef BWD
    probe_add(DM_PROBE_ATTN_BWD_MFMA, 4);
    DM_LAUNCH_CHECK("attention_backward: MFMA launch");
    return DM_OK;
}

}  // namespace dm
