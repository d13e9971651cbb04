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

// ------------------------------------------------------------------------------------------
// dK, dV
// ------------------------------------------------------------------------------------------

template <int D>
struct BwdStrides {
    static constexpr int ROW = D + 8;  // rows read by ds_read_b128
    static constexpr int TR = D + 32;  // rows read by ds_read_b64_tr_b16
};

template <int D>
struct DkdvSmem {
    uint4 q[kQTile * BwdStrides<D>::ROW / 8];
    uint4 qt[kQTile * BwdStrides<D>::TR / 8];
    uint4 g[kQTile * BwdStrides<D>::ROW / 8];
    uint4 gt[kQTile * BwdStrides<D>::TR / 8];
    float lse2[kQTile], delta[kQTile];
    int32_t rlo[kQTile], rhi[kQTile];
};

template <int DT, int D, bool PAD>
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
    constexpr int RS = BwdStrides<D>::ROW, TS = BwdStrides<D>::TR;
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
    const int32_t j0 = (int32_t)(kb * kKvBlock);
    const int32_t key = j0 + wave * 32 + col;  // this lane's key
    const bool kvalid = key < Tk;
    const bool kpad = PAD && kvalid && m.pad[b * Tk + key];
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
    const int32_t j1 = j0 + kKvBlock < Tk ? j0 + kKvBlock : (int32_t)Tk;
    auto sees = [&](int64_t t) -> bool { return tr[t * 4] < j1 && tr[t * 4 + 1] > j0; };

    // staging: Q and dO tiles in 16-byte chunks (buffer loads whose range ends at the last
    // query row), written to a row copy and a transposed-read copy
    constexpr int CPR = D / 8, NCH = kQTile * CPR / 256, RSTEP = 256 / CPR;
    const int crow = tid / CPR, ccol = tid % CPR;
    const uint32_t qrow_bytes = (uint32_t)(Hq * D * 2);
    const uint32_t qbytes = (uint32_t)(((Tq - 1) * Hq + 1) * D * 2);
    const uint32_t goff = crow * qrow_bytes + ccol * 16;
    uint4 qreg[NCH], greg[NCH];
    __amdgpu_buffer_rsrc_t qrs, grs;
    auto load = [&](int64_t h, int64_t t) {
        qrs = make_rsrc(q + (b * Tq * Hq + h) * D, qbytes);
        grs = make_rsrc(d_o + (b * Tq * Hq + h) * D, qbytes);
        const uint32_t base = (uint32_t)(t * kQTile) * qrow_bytes + goff;
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            const uint32_t off = base + u * RSTEP * qrow_bytes;
            qreg[u] = buf_load16(qrs, off);
            greg[u] = buf_load16(grs, off);
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
        for (int u = 0; u < NCH; u++) {
            const int r = crow + u * RSTEP;
            sm.q[r * (RS / 8) + ccol] = qreg[u];
            sm.qt[r * (TS / 8) + ccol] = qreg[u];
            sm.g[r * (RS / 8) + ccol] = greg[u];
            sm.gt[r * (TS / 8) + ccol] = greg[u];
        }
        if (tid < kQTile) {
            sm.lse2[tid] = st_lse;
            sm.delta[tid] = st_delta;
            sm.rlo[tid] = st_lo;
            sm.rhi[tid] = st_hi;
        }
    };
    const uint16_t *sq = (const uint16_t *)sm.q, *sqt = (const uint16_t *)sm.qt;
    const uint16_t *sg = (const uint16_t *)sm.g, *sgt = (const uint16_t *)sm.gt;

    // the (head, tile) steps: the group's query heads, each over the tiles that see the keys
    int64_t hh = kh * group, tt = 0;
    const int64_t hend = (kh + 1) * group;
    auto advance = [&](int64_t &h, int64_t &t) {
        while (h < hend) {
            while (t < ntiles && !sees(t)) t++;
            if (t < ntiles) return;
            h++;
            t = 0;
        }
    };
    const bool any_key = j0 < Tk;
    if (any_key) advance(hh, tt);
    if (any_key && hh < hend) {
        load(hh, tt);
        load_rows(hh, tt);
    }
    while (any_key && hh < hend) {
        const int64_t t = tt;
        __syncthreads();
        store();
        __syncthreads();
        // next step's loads, in flight during this step's products
        tt++;
        advance(hh, tt);
        if (hh < hend) {
            load(hh, tt);
            load_rows(hh, tt);
        }
        const int32_t *r = tr + t * 4;
        const bool masked = PAD || r[2] > j0 || r[3] < j0 + kKvBlock;
#pragma unroll
        for (int qs = 0; qs < kQTile / 32; qs++) {
            // S and dP for 32 queries x this wavefront's 32 keys
            f32x16_t s, dp;
#pragma unroll
            for (int i = 0; i < 16; i++) s[i] = dp[i] = 0.f;
            const uint16_t *qa = sq + (qs * 32 + col) * RS + half * 8;
            const uint16_t *ga = sg + (qs * 32 + col) * RS + half * 8;
#pragma unroll
            for (int st = 0; st < KSTEPS; st++) {
                Frag8 a;
                a.u = *(const uint4 *)(qa + st * 16);
                s = mfma32<DT>(a, kf[st], s);
                a.u = *(const uint4 *)(ga + st * 16);
                dp = mfma32<DT>(a, vf[st], dp);
            }
            // P = exp2(S c - lse2), dS = P (dP - delta); element i is query
            //   32 qs + 8 (i / 4) + 4 h + i % 4, four consecutive rows per i / 4
            Frag8 pf[2], df[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                float p[8], ds[8];
#pragma unroll
                for (int g4 = 0; g4 < 2; g4++) {
                    const int r0 = qs * 32 + (2 * u + g4) * 8 + half * 4;
                    const float4 l4 = *(const float4 *)(sm.lse2 + r0);
                    const float4 d4 = *(const float4 *)(sm.delta + r0);
                    const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
                    const float dl[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int i = 8 * u + 4 * g4 + e;
                        float x = fast_exp2(fmaf(s[i], c2, -lv[e]));
                        if (masked) {
                            const bool vis = key >= sm.rlo[r0 + e] && key < sm.rhi[r0 + e] && !kpad;
                            x = vis ? x : 0.f;
                        }
                        p[4 * g4 + e] = x;
                        ds[4 * g4 + e] = x * (dp[i] - dl[e]);
                    }
                }
                pf[u].u = make_uint4(pack2<DT>(p[0], p[1]), pack2<DT>(p[2], p[3]),
                                     pack2<DT>(p[4], p[5]), pack2<DT>(p[6], p[7]));
                df[u].u = make_uint4(pack2<DT>(ds[0], ds[1]), pack2<DT>(ds[2], ds[3]),
                                     pack2<DT>(ds[4], ds[5]), pack2<DT>(ds[6], ds[7]));
            }
            // dV += P^T dO, dK += dS^T Q: A = (row key, k = query) from the products' output,
            // B = (k = query, col = d) by transposed reads of the row-major tiles
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int dt = 0; dt < DT32; dt++) {
                    const Frag8 bg = lds_tr_frag(sgt, TS, qs * 32 + u * 16, dt * 32, lane);
                    const Frag8 bq = lds_tr_frag(sqt, TS, qs * 32 + u * 16, dt * 32, lane);
                    dva[dt] = mfma32<DT>(pf[u], bg, dva[dt]);
                    dka[dt] = mfma32<DT>(df[u], bq, dka[dt]);
                }
        }
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
            const uint32_t kv2 = pack2<DT>(dka[dt][i] * scale, dva[dt][i]);
            dk[off] = (uint16_t)(kv2 & 0xffffu);
            dv[off] = (uint16_t)(kv2 >> 16);
        }
}

// ------------------------------------------------------------------------------------------
// dQ
// ------------------------------------------------------------------------------------------

template <int D>
struct DqSmem {
    uint4 k[kDqN * BwdStrides<D>::ROW / 8];
    uint4 v[kDqN * BwdStrides<D>::ROW / 8];
    uint4 kt[kDqN * BwdStrides<D>::TR / 8];
    int32_t lo[4], hi[4], flo[4], fhi[4];
};

template <int DT, int D, bool PAD>
__global__ __launch_bounds__(256, 1) void bwd_dq(MaskInfo m, int64_t B, int64_t Hq, int64_t Hkv,
                                                 float scale, const uint16_t *__restrict__ q,
                                                 const uint16_t *__restrict__ k,
                                                 const uint16_t *__restrict__ v,
                                                 const uint16_t *__restrict__ d_o,
                                                 const float *__restrict__ delta, BwdWs w,
                                                 uint16_t *__restrict__ dq) {
    using Sm = DqSmem<D>;
    constexpr int RS = BwdStrides<D>::ROW, TS = BwdStrides<D>::TR;
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
    const float nlse = -lse2;
    const int32_t kvstride = (int32_t)(Hkv * D);
    const uint32_t kvbytes = (uint32_t)(((Tk - 1) * Hkv + 1) * D * 2);
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(k + (b * Tk * Hkv + kh) * D, kvbytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(v + (b * Tk * Hkv + kh) * D, kvbytes);
    const uint8_t *pad = PAD ? m.pad + b * Tk : nullptr;

    constexpr int CPR = D / 8, NCH = kDqN * CPR / 256, RSTEP = 256 / CPR;
    const int crow = tid / CPR, ccol = tid % CPR;
    const uint32_t goff = (uint32_t)(crow * kvstride + ccol * 8) * 2;
    uint4 kreg[NCH], vreg[NCH];
    auto load_tile = [&](int32_t j0) {
        const uint32_t base = (uint32_t)j0 * (uint32_t)kvstride * 2 + goff;
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            const uint32_t off = base + (uint32_t)(u * RSTEP * kvstride * 2);
            kreg[u] = buf_load16(krs, off);
            vreg[u] = buf_load16(vrs, off);
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            const int r = crow + u * RSTEP;
            sm.k[r * (RS / 8) + ccol] = kreg[u];
            sm.kt[r * (TS / 8) + ccol] = kreg[u];
            sm.v[r * (RS / 8) + ccol] = vreg[u];
        }
    };
    const uint16_t *sk = (const uint16_t *)sm.k, *sv = (const uint16_t *)sm.v;
    const uint16_t *skt = (const uint16_t *)sm.kt;

    if (kv_lo < kv_hi) load_tile(kv_lo);
    for (int32_t j0 = kv_lo; j0 < kv_hi; j0 += kDqN) {
        __syncthreads();
        store_tile();
        __syncthreads();
        if (j0 + kDqN < kv_hi) load_tile(j0 + kDqN);
        const bool masked = PAD || j0 < full_lo || j0 + kDqN > full_hi;
        Frag8 df[2][2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            f32x16_t s, dp;
#pragma unroll
            for (int i = 0; i < 16; i++) s[i] = dp[i] = 0.f;
            const uint16_t *ka = sk + (t * 32 + col) * RS + half * 8;
            const uint16_t *va = sv + (t * 32 + col) * RS + half * 8;
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
                    float p = fast_exp2(fmaf(s[i], c2, nlse));
                    if (masked) {
                        const int32_t j = j0 + t * 32 + (i / 4) * 8 + half * 4 + (i % 4);
                        bool vis = j >= lo && j < hi;
                        if constexpr (PAD) vis = vis && !pad[j];
                        p = vis ? p : 0.f;
                    }
                    ds[e] = p * (dp[i] - dl);
                }
                df[t][u].u = make_uint4(pack2<DT>(ds[0], ds[1]), pack2<DT>(ds[2], ds[3]),
                                        pack2<DT>(ds[4], ds[5]), pack2<DT>(ds[6], ds[7]));
            }
        }
        // dQ^T += K^T dS^T: A = K^T by transposed reads of the row-major K tile
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int dt = 0; dt < DT32; dt++) {
                    const Frag8 a = lds_tr_frag(skt, TS, t * 32 + u * 16, dt * 32, lane);
                    acc[dt] = mfma32<DT>(a, df[t][u], acc[dt]);
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
           d->tq < (1ll << 30) && d->tk < (1ll << 30) && scale_of(d) > 0.f &&
           d->tk * d->hkv * d->d * 2 < (1ll << 31) && d->tq * d->hq * d->d * 2 < (1ll << 31);
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
    if (m.pad) {                                                                               \
        { KernelTimer t1(DM_KERNEL_ATTN_BWD_DKDV, st);                                       \
        bwd_dkdv<DT, DD, true><<<(unsigned)nb_kv, 256, 0, st>>>(m, d->b, d->hq, d->hkv, scale, \
                                                                qq, kk, vv, gg, delta, w,      \
                                                                (uint16_t *)dk, (uint16_t *)dv); } \
        { KernelTimer t2(DM_KERNEL_ATTN_BWD_DQ, st);                                         \
        bwd_dq<DT, DD, true><<<(unsigned)nb_q, 256, 0, st>>>(m, d->b, d->hq, d->hkv, scale, qq,  \
                                                             kk, vv, gg, delta, w,             \
                                                             (uint16_t *)dq); }                \
    } else {                                                                                   \
        { KernelTimer t1(DM_KERNEL_ATTN_BWD_DKDV, st);                                       \
        bwd_dkdv<DT, DD, false><<<(unsigned)nb_kv, 256, 0, st>>>(m, d->b, d->hq, d->hkv, scale, \
                                                                 qq, kk, vv, gg, delta, w,     \
                                                                 (uint16_t *)dk, (uint16_t *)dv); } \
        { KernelTimer t2(DM_KERNEL_ATTN_BWD_DQ, st);                                         \
        bwd_dq<DT, DD, false><<<(unsigned)nb_q, 256, 0, st>>>(m, d->b, d->hq, d->hkv, scale, qq, \
                                                              kk, vv, gg, delta, w,            \
                                                              (uint16_t *)dq); }               \
    }
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
