// MFMA attention forward for gfx950: bf16/f16 inputs, f32 accumulation, head
// width 64 or 128 (the flash-attention forward of crates/dash-ops/src/attention/kernels.rs:683-997).
//
// A workgroup of 8 wavefronts takes 256 queries of one head, each wavefront 32 of them, and
// sweeps the keys the workgroup sees in tiles of 64. Wavefronts w and w + 4 run on one SIMD and
// are kept half a step apart by the workgroup's barriers: while one runs its products, the other
// runs its softmax, so the SIMD's matrix unit and vector unit work at the same time. Per step j
// and wavefront, between two barriers:
//   products   S^T_j = K_j Q^T (A = K rows from LDS, B = the wavefront's queries in registers)
//              and O^T += V_{j-1}^T P^T_{j-1} (A = V^T by transposed LDS reads, B = P^T of the
//              previous step, still in registers), at raised wave priority;
//   softmax    the online softmax of S^T_j: maxima, the lazy rescale of O, P^T_j as bf16 B
//              fragments; plus this thread's share of staging the next K and V tiles.
// Wavefronts 0-3 run products then softmax in each step, wavefronts 4-7 softmax (of the previous
// step) then products. K_j and V_{j-1} are the tiles in use during step j; K_{j+1} and V_j are
// staged into the other LDS slots during step j, from registers loaded one step earlier.
// A wavefront skips the products and softmax of a tile none of its queries sees (it still takes
// part in every barrier); the per-element mask runs only on tiles its rows' intervals cut.
#include <string>

#include "attention_kernels.h"
#include "mfma.h"

namespace dm {

// queries per workgroup: 32 per wavefront, 8 wavefronts (ping-pong pairs) at D 64 and 128, 4 at
// D 256 (one per SIMD: 32 queries' O^T over 256 columns and their Q fragments take 192
// registers, more than two wavefronts per SIMD hold)
template <int D>
constexpr int fwd_waves() { return D == 256 ? 4 : 8; }
constexpr int kFwdN = 64;   // keys per tile

// Row strides (elements) of the LDS tiles: K rows are read along D by ds_read_b128 (16 lanes on
// 16 consecutive rows, conflict-free at 16 mod 256 bytes); V rows transposed by
// ds_read_b64_tr_b16 (conflict-free at 64 mod 256 bytes).
template <int D>
struct FwdStrides {
    static constexpr int K = D + 8;
    static constexpr int V = D + 32;
};

template <int D>
struct FwdSmem {
    uint4 k[2][kFwdN * FwdStrides<D>::K / 8];
    uint4 v[2][kFwdN * FwdStrides<D>::V / 8];
    int32_t lo[8], hi[8], flo[8], fhi[8];
};

// The per-tile rescale is skipped until a row's maximum grows by more than 2^8 over the one its
// exponentials are taken against (p stays below 256; the normalisation uses the same reference).
constexpr float kRescaleThreshold = 8.f;

#ifdef DM_TRACE_FWD
// profiling aid (built only with -DDM_TRACE_FWD): per-step clock stamps of wavefronts 0 and 4 of
// one workgroup
__device__ uint64_t dm_trace_fwd[2][256][4];
#define DM_FSTAMP(step, k)                                                                      \
    do {                                                                                       \
        if (work == DM_TRACE_FWD && (wave & 3) == 0 && lane == 0 && (step) < 256)             \
            dm_trace_fwd[wave >> 2][step][k] = __builtin_readcyclecounter();                   \
    } while (0)
#else
#define DM_FSTAMP(step, k) \
    do {                   \
    } while (0)
#endif

template <int DT, int D, bool PAD>
__global__ __launch_bounds__(64 * fwd_waves<D>(), 1) void attn_fwd_mfma(MaskInfo m, int64_t B, int64_t Hq,
                                                      int64_t Hkv, float scale, AttnStrides sd,
                                                      const uint16_t *__restrict__ q,
                                                      const uint16_t *__restrict__ k,
                                                      const uint16_t *__restrict__ v,
                                                      uint16_t *__restrict__ o,
                                                      float *__restrict__ lse) {
    constexpr int KS = FwdStrides<D>::K, VS = FwdStrides<D>::V;
    __shared__ FwdSmem<D> sm;
    constexpr int KSTEPS = D / 16;  // k-steps of S^T over the head dimension
    constexpr int DT32 = D / 32;    // 32-row tiles of O^T
    constexpr int NW = fwd_waves<D>(), NT = 64 * NW, kFwdM = 32 * NW;
    const int64_t Tq = m.tq, Tk = m.tk;
    const int64_t ntiles = (Tq + kFwdM - 1) / kFwdM;
    const int64_t nwork = ntiles * Hq * B;
    const int64_t work = blockIdx.x;
    if (work >= nwork) return;
    // the key-value head is the fastest index (consecutive workgroups go to consecutive XCDs: with
    // Hkv = 8 an XCD holds one key-value head's keys in its L2), then the query head of the group,
    // then the query tiles from the longest (last) down, then the batch row
    const int64_t kh = work % Hkv;
    const int64_t h = kh * (Hq / Hkv) + (work / Hkv) % (Hq / Hkv);
    const int64_t tile = ntiles - 1 - (work / Hq) % ntiles;
    const int64_t b = work / (Hq * ntiles);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool first = NW == 4 || wave < 4;  // products first in each step
    const int col = lane & 31, half = lane >> 5;
    const int64_t qi = tile * kFwdM + wave * 32 + col;  // this lane's query row
    const bool qvalid = qi < Tq;

    int64_t lo64 = 0, hi64 = 0;
    if (qvalid) row_bounds(m, qi, &lo64, &hi64);
    const int32_t lo = (int32_t)lo64, hi = (int32_t)hi64;
    {
        // this wavefront's union of its rows' intervals, and the keys all of them see (a row
        // that sees nothing forces the mask on every tile)
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
    int32_t kv_lo = INT32_MAX, kv_hi = INT32_MIN;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        kv_lo = min(kv_lo, sm.lo[w]);
        kv_hi = max(kv_hi, sm.hi[w]);
    }
    kv_lo = __builtin_amdgcn_readfirstlane(kv_lo);
    kv_hi = __builtin_amdgcn_readfirstlane(kv_hi);
    const int32_t my_lo = __builtin_amdgcn_readfirstlane(sm.lo[wave]);
    const int32_t my_hi = __builtin_amdgcn_readfirstlane(sm.hi[wave]);
    const int32_t my_flo = __builtin_amdgcn_readfirstlane(sm.flo[wave]);
    const int32_t my_fhi = __builtin_amdgcn_readfirstlane(sm.fhi[wave]);
    const int32_t nt = kv_lo < kv_hi ? (kv_hi - kv_lo + kFwdN - 1) / kFwdN : 0;

    // this wavefront's queries as the B operand: col = query, k = head dimension
    Frag8 qf[KSTEPS];
    {
        const uint16_t *qp = q + b * sd.q.b + qi * sd.q.t + h * sd.q.h + half * 8;
#pragma unroll
        for (int s = 0; s < KSTEPS; s++)
            qf[s].u = qvalid ? *(const uint4 *)(qp + s * 16) : make_uint4(0, 0, 0, 0);
        // wait for them here (s_waitcnt vmcnt(0)), before the tile loads below: issued after
        // those, they would leave a wait for every load in flight in the loop
        __builtin_amdgcn_s_waitcnt(0x0F70);
    }

    f32x16_t acc[DT32];
#pragma unroll
    for (int t = 0; t < DT32; t++) acc[t] = zero16();
    // mc: the reference the exponentials are taken against (max raw score x scale x log2 e);
    // lrow: this lane's partial sum of the exponentials
    float mc = -INFINITY, lrow = 0.f;
    const float c2 = scale * 1.4426950408889634f;

    // staging: 16-byte chunks of one K and one V tile per thread, by buffer loads whose range
    // ends at the last key (rows past it read zeros)
    // (row strides in elements; the host checked that every byte range fits 32 bits)
    const int32_t kstride = (int32_t)sd.k.t, vstride = (int32_t)sd.v.t;
    const uint32_t kbytes = (uint32_t)(((Tk - 1) * sd.k.t + D) * 2);
    const uint32_t vbytes = (uint32_t)(((Tk - 1) * sd.v.t + D) * 2);
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(k + b * sd.k.b + kh * sd.k.h, kbytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(v + b * sd.v.b + kh * sd.v.h, vbytes);
    const uint8_t *pad = PAD ? m.pad + b * Tk : nullptr;
    constexpr int CPR = D / 8;              // chunks per row
    constexpr int NCH = kFwdN * CPR / NT;    // chunks per thread per tensor
    constexpr int RSTEP = NT / CPR;         // rows between a thread's chunks
    const int crow = tid / CPR, ccol = tid % CPR;
    const uint32_t koff = (uint32_t)(crow * kstride + ccol * 8) * 2;
    const uint32_t voff = (uint32_t)(crow * vstride + ccol * 8) * 2;
    uint4 rk[NCH], rv[NCH];
    auto tile_key = [&](int32_t j) { return kv_lo + (j < nt ? j : 0) * kFwdN; };
    auto load_k = [&](int32_t j) __attribute__((always_inline)) {
        const uint32_t base = (uint32_t)tile_key(j) * (uint32_t)kstride * 2 + koff;
#pragma unroll
        for (int u = 0; u < NCH; u++) rk[u] = buf_load16(krs, base + (uint32_t)(u * RSTEP * kstride * 2));
    };
    auto load_v = [&](int32_t j) __attribute__((always_inline)) {
        const uint32_t base = (uint32_t)tile_key(j) * (uint32_t)vstride * 2 + voff;
#pragma unroll
        for (int u = 0; u < NCH; u++) rv[u] = buf_load16(vrs, base + (uint32_t)(u * RSTEP * vstride * 2));
    };
    auto store_k = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NCH; u++) sm.k[slot][(crow + u * RSTEP) * (KS / 8) + ccol] = rk[u];
    };
    auto store_v = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NCH; u++) sm.v[slot][(crow + u * RSTEP) * (VS / 8) + ccol] = rv[u];
    };

    // per-wavefront tile tests (wavefront-uniform)
    auto sees = [&](int32_t j) {
        const int32_t j0 = kv_lo + j * kFwdN;
        return j >= 0 && j < nt && my_lo < my_hi && j0 < my_hi && j0 + kFwdN > my_lo;
    };
    auto cut = [&](int32_t j) {
        const int32_t j0 = kv_lo + j * kFwdN;
        return PAD || j0 < my_flo || j0 + kFwdN > my_fhi;
    };

    f32x16_t s[2];      // S^T of the current tile: two 32-key row tiles
    Frag8 pf[2][2];     // P^T of the previous tile as B fragments

    // products of step j: S^T_j (if this wavefront sees tile j) and O^T += V^T_{j-1} P^T_{j-1}
    // (if it saw tile j - 1), at raised wave priority
    auto products = [&](int32_t j) __attribute__((always_inline)) {
        __builtin_amdgcn_s_setprio(1);
        if (sees(j)) {
            const uint16_t *sk = (const uint16_t *)sm.k[j & 1];
#pragma unroll
            for (int t = 0; t < 2; t++) s[t] = zero16();
#pragma unroll
            for (int st = 0; st < KSTEPS; st++)
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    Frag8 a;
                    a.u = *(const uint4 *)(sk + (t * 32 + col) * KS + half * 8 + st * 16);
                    s[t] = mfma32<DT>(a, qf[st], s[t]);
                }
        }
        // (the scheduler would otherwise hoist every fragment read of both products to the top)
        __builtin_amdgcn_sched_barrier(0);
        if (sees(j - 1)) {
            // key order 32 t + 16 u + 8 (e / 4) + 4 h + e % 4 in slot e of lane half h of step
            // (t, u): the output layout of S^T
            const uint16_t *sv = (const uint16_t *)sm.v[(j - 1) & 1];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int u = 0; u < 2; u++)
#pragma unroll
                    for (int dt = 0; dt < DT32; dt++) {
                        const Frag8 a = lds_tr_frag(sv, VS, t * 32 + u * 16, dt * 32, lane);
                        acc[dt] = mfma32<DT>(a, pf[t][u], acc[dt]);
                    }
        }
        __builtin_amdgcn_s_setprio(0);
    };

    // softmax of tile jj (this wavefront sees it): mask, maxima, lazy rescale, P^T fragments
    auto softmax = [&](int32_t jj) __attribute__((always_inline)) {
        const int32_t j0 = kv_lo + jj * kFwdN;
        if (cut(jj)) {
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
    };

    // Staging: thread shares of the tiles, from registers loaded one step earlier. Wavefronts 0-3
    // store K_{j+1} and V_j during their softmax of step j, wavefronts 4-7 (half a step later)
    // K_{j+2} and V_{j+1}; each tile's two shares are in place before its first reader's step.
    const int32_t ahead = first ? 0 : 1;
    auto stage = [&](int32_t j) __attribute__((always_inline)) {
        store_k((j + 1 + ahead) & 1);
        store_v((j + ahead) & 1);
        load_k(j + 2 + ahead);
        load_v(j + 1 + ahead);
    };

    // prologue: K_0 into its slot, this thread's shares of K_1 and V_0 into the registers
    if (nt > 0) {
        load_k(0);
        store_k(0);
        load_k(1);
        load_v(0);
    }
    __syncthreads();
    // Every wavefront runs steps j = 0 .. nt as [products of step j | barrier | softmax of tile j,
    // staging | barrier]. Wavefronts 4-7 first stage their shares of K_1 and V_0 and pass one
    // barrier, so they run half a step behind wavefronts 0-3, which pass one barrier at the end.
    if (!first) {
        if (nt > 0) stage(-1);
        __syncthreads();
    }
    for (int32_t j = 0; j <= nt; j++) {
        DM_FSTAMP(j, 0);
        products(j);
        DM_FSTAMP(j, 1);
        __syncthreads();
        DM_FSTAMP(j, 2);
        if (sees(j)) softmax(j);
        if (j < nt) stage(j);
        DM_FSTAMP(j, 3);
        __syncthreads();
    }
    if (first) __syncthreads();

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

// Whether the 16-bit kernels' buffer loads reach `rows` rows of `x` (a row every x.t elements,
// D wide) with 32-bit byte offsets from one (batch, head) base.
bool rows_fit_32bit(const Strd &x, int64_t rows, int64_t d) {
    return rows <= 0 || ((rows - 1) * x.t + d) * 2 < (1ll << 31);
}

bool mfma_fwd_takes(const dm_attention_desc *d, const void *q, const void *k, const void *v) {
    // a positive scale keeps the maximum of the raw scores the maximum of the scaled ones;
    // buffer loads take 32-bit byte offsets within one (batch row, head)'s keys and values;
    // 16-byte vector loads need 16-byte rows and bases
    const AttnStrides s = attn_strides(d);
    return (d->dtype == DM_BF16 || d->dtype == DM_F16) &&
           (d->d == 64 || d->d == 128 || d->d == 256) && d->tq < (1ll << 30) &&
           d->tk < (1ll << 30) && scale_of(d) > 0.f && rows_fit_32bit(s.k, d->tk, d->d) && rows_fit_32bit(s.v, d->tk, d->d) &&
           strides_16b(s.q) && strides_16b(s.k) && strides_16b(s.v) && aligned_16b(q) &&
           aligned_16b(k) && aligned_16b(v);
}

#ifdef DM_TRACE_FWD
extern "C" int dm_debug_trace_fwd(void *host, size_t bytes) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(dm_trace_fwd), bytes) == hipSuccess ? 0 : 1;
}
#endif

int launch_attn_fwd_mfma(const MaskInfo &m, const dm_attention_desc *d, float scale,
                         const void *q, const void *k, const void *v, void *o, float *lse,
                         hipStream_t st) {
    const int nw = d->d == 256 ? fwd_waves<256>() : fwd_waves<128>();
    const int64_t per = 32 * nw;  // queries per workgroup
    const int64_t ntiles = (d->tq + per - 1) / per;
    const int64_t nwork = ntiles * d->hq * d->b;
    const int64_t nblocks = (nwork + 7) / 8 * 8;
    if (nblocks >= (1ll << 31)) return refuse("attention: too many query tiles");
    dim3 grid((unsigned)nblocks), block(64 * nw);
    const uint16_t *qq = (const uint16_t *)q, *kk = (const uint16_t *)k, *vv = (const uint16_t *)v;
    uint16_t *oo = (uint16_t *)o;
    const AttnStrides sd = attn_strides(d);
#define FWD(DT, DD)                                                                           \
    if (m.pad)                                                                                \
        attn_fwd_mfma<DT, DD, true><<<grid, block, 0, st>>>(m, d->b, d->hq, d->hkv, scale, sd,  \
                                                          qq, kk, vv, oo, lse);              \
    else                                                                                      \
        attn_fwd_mfma<DT, DD, false><<<grid, block, 0, st>>>(m, d->b, d->hq, d->hkv, scale, sd, \
                                                           qq, kk, vv, oo, lse)
    {
        KernelTimer timer(DM_KERNEL_ATTN_FWD, st);
        if (d->dtype == DM_BF16) {
            if (d->d == 64) { FWD(DM_BF16, 64); } else if (d->d == 128) { FWD(DM_BF16, 128); } else { FWD(DM_BF16, 256); }
        } else {
            if (d->d == 64) { FWD(DM_F16, 64); } else if (d->d == 128) { FWD(DM_F16, 128); } else { FWD(DM_F16, 256); }
        }
    }
#undef FWD
    probe_add(DM_PROBE_ATTN_FWD_MFMA);
    DM_LAUNCH_CHECK("attention: MFMA forward launch");
    return DM_OK;
}

}  // namespace dm
