// MFMA attention backward at head width 256: the dK/dV kernel (bwd_dkdv_w4). A translation unit
// of its own so that it is scheduled with the compiler's occupancy-driven iterative strategy,
// which suits its single-role wavefronts better than the memory-clause strategy the other
// attention kernels take (crates/dash-ops/src/attention/kernels.rs:999-2058).
#include "attention_bwd.h"
#include "mfma.h"

namespace dm {

// ------------------------------------------------------------------------------------------
// Head width 256: single-role wavefronts
// ------------------------------------------------------------------------------------------
//
// At D = 256 a wavefront's 32 keys need dK and dV accumulators of 128 registers each, and the
// products' outputs share the accumulator registers with them: both gradients at once do not
// fit beside the S and dP outputs. The gradients are then two passes of one kernel body, each
// workgroup 4 wavefronts (one per SIMD) taking 32 keys each through every step:
//   dV pass: S = Q K^T, P, dV += P^T dO                      (32 products of 32x32x16 a step)
//   dK pass: S = Q K^T, P, dP = dO V^T, dS = P (dP - delta), dK += dS^T Q     (48 a step)
// (80 products against the 64 of a single pass: S is computed twice). The tiles a pass reads
// rotate through two LDS slots, staged one step ahead through registers. The work list, the
// schedule ring and the query-head split are the 8-wavefront kernel's.
constexpr int kDkdvDV = 0, kDkdvDK = 1;

template <int D>
struct Dkdv4Smem {
    DkdvSlot<D> slot[2];
    int4 sched[kDkdvRing];
};

template <int DT, int D, bool PAD, int MODE>
__device__ __forceinline__ void dkdv_w4_pass(Dkdv4Smem<D> &sm, const int64_t work, MaskInfo m,
                                             int64_t B, int64_t Hq, int64_t Hkv, float scale,
                                             AttnStrides sd, const uint16_t *__restrict__ q,
                                             const uint16_t *__restrict__ k,
                                             const uint16_t *__restrict__ v,
                                             const uint16_t *__restrict__ d_o,
                                             const float *__restrict__ delta, BwdWs w,
                                             uint16_t *__restrict__ out) {
    constexpr bool DK = MODE == kDkdvDK;
    constexpr int RS = BwdStrides<D>::ROW, TS = BwdStrides<D>::TR;
    constexpr int KSTEPS = D / 16, DT32 = D / 32;
    const int64_t Tq = m.tq, Tk = m.tk;
    const int64_t nkb = (Tk + kKvBlock - 1) / kKvBlock;
    const int hs = w.hsplit;
    const int64_t kh = work % Hkv, part = (work / Hkv) % hs;
    const int64_t kb = (work / (Hkv * hs)) % nkb, b = work / (Hkv * hs * nkb);
    const int64_t group = Hq / Hkv;
    const int64_t h_first = kh * group + part * (group / hs);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kw = wave;
    const int col = lane & 31, half = lane >> 5;
    const int32_t j0 = (int32_t)(kb * kKvBlock);
    const int32_t key = j0 + kw * 32 + col;
    const bool kvalid = key < Tk;
    const bool kpad = PAD && kvalid && m.pad[b * Tk + key];
    const int32_t mkey = kpad ? -1 : key;
    const float c2 = scale * 1.4426950408889634f;

    // K (and, for dK, V) of this lane's key as B operands (col = key, k = head dim)
    Frag8 bk[KSTEPS], bv[DK ? KSTEPS : 1];
    {
        const uint16_t *kp = k + b * sd.k.b + (int64_t)key * sd.k.t + kh * sd.k.h + half * 8;
        const uint16_t *vp = v + b * sd.v.b + (int64_t)key * sd.v.t + kh * sd.v.h + half * 8;
#pragma unroll
        for (int st = 0; st < KSTEPS; st++) {
            bk[st].u = kvalid ? *(const uint4 *)(kp + st * 16) : make_uint4(0, 0, 0, 0);
            if constexpr (DK) bv[st].u = kvalid ? *(const uint4 *)(vp + st * 16) : make_uint4(0, 0, 0, 0);
        }
    }
    f32x16_t acc[DT32];
#pragma unroll
    for (int t = 0; t < DT32; t++) acc[t] = zero16();

    const int64_t ntiles = (Tq + kDkdvStep - 1) / kDkdvStep;
    const int32_t *tr = w.trange + b * ntiles * 4;
    const int32_t j1 = j0 + kKvBlock < Tk ? j0 + kKvBlock : (int32_t)Tk;
    const int32_t hend = (int32_t)(h_first + group / hs);
    struct TileIter {
        int32_t h, t, c0;
        uint64_t pending, cut;
        bool masked;
    };
    auto scan = [&](TileIter &it) {
        const int32_t tt = it.c0 + lane;
        const int4 r = *(const int4 *)(tr + (tt < ntiles ? tt : ntiles - 1) * 4);
        const bool in = tt < ntiles;
        const bool see = in & (r.x < j1) & (r.y > j0);
        const bool pcut = PAD | (r.z > j0) | (r.w < j0 + kKvBlock);
        it.pending = __ballot(see);
        it.cut = __ballot(pcut);
    };
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
    TileIter it;
    auto publish = [&](const int kk) __attribute__((always_inline)) {
        if (lane == 0)
            sm.sched[kk % kDkdvRing] = make_int4(it.h, it.t, it.masked ? 1 : 0, it.h < hend ? 1 : 0);
        if (it.h < hend) next(it);
    };
    if (wave == 0) {
        it.h = (int32_t)h_first;
        it.c0 = 0;
        it.t = -1;
        if (j0 >= Tk) {
            it.h = hend;
        } else {
            scan(it);
            next(it);
        }
        for (int kk = 0; kk < 4; kk++) publish(kk);
    }
    __syncthreads();
    struct Entry {
        int32_t h, t;
        bool masked, valid;
    };
    auto entry = [&](const int kk) __attribute__((always_inline)) -> Entry {
        const int4 e = sm.sched[kk % kDkdvRing];
        Entry x;
        x.h = __builtin_amdgcn_readfirstlane(e.x);
        x.t = __builtin_amdgcn_readfirstlane(e.y);
        x.masked = __builtin_amdgcn_readfirstlane(e.z) != 0;
        x.valid = __builtin_amdgcn_readfirstlane(e.w) != 0;
        return x;
    };

    // staging: a step's Q and dO rows, 16-byte chunks over the 256 threads
    constexpr int CPR = D / 8, NCH = kDkdvStep * CPR / 256, RSTEP = 256 / CPR;
    const int crow = tid / CPR, ccol = tid % CPR;
    const uint32_t qrow_bytes = (uint32_t)(sd.q.t * 2), grow_bytes = (uint32_t)(sd.g.t * 2);
    const uint32_t qbytes = (uint32_t)(((Tq - 1) * sd.q.t + D) * 2);
    const uint32_t gbytes = (uint32_t)(((Tq - 1) * sd.g.t + D) * 2);
    const uint32_t mbytes = (uint32_t)(((Tq - 1) * Hq + 1) * 4);
    const __amdgpu_buffer_rsrc_t lrs = make_rsrc(w.rlo + b * Tq, (uint32_t)(Tq * 4));
    const __amdgpu_buffer_rsrc_t hrs = make_rsrc(w.rhi + b * Tq, (uint32_t)(Tq * 4));
    struct Stage {
        uint4 q[NCH], g[NCH];
        float lse, delta;
        int32_t lo, hi;
    };
    Stage stg;
    auto load = [&](int64_t h, int64_t t) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t qrs = make_rsrc(q + b * sd.q.b + h * sd.q.h, qbytes);
        const __amdgpu_buffer_rsrc_t grs = make_rsrc(d_o + b * sd.g.b + h * sd.g.h, gbytes);
        const uint32_t i0 = (uint32_t)(t * kDkdvStep);
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            const uint32_t r = i0 + (uint32_t)(crow + u * RSTEP);
            stg.q[u] = buf_load16(qrs, r * qrow_bytes + ccol * 16);
            stg.g[u] = buf_load16(grs, r * grow_bytes + ccol * 16);
        }
        const uint32_t i = i0 + (tid & (kDkdvStep - 1));
        const __amdgpu_buffer_rsrc_t srs = make_rsrc(w.lse2 + b * Tq * Hq + h, mbytes);
        stg.lse = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(srs, i * (uint32_t)Hq * 4, 0, 0));
        if constexpr (DK) {
            const __amdgpu_buffer_rsrc_t drs = make_rsrc(delta + b * Tq * Hq + h, mbytes);
            stg.delta = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(drs, i * (uint32_t)Hq * 4, 0, 0));
        }
        stg.lo = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(lrs, i * 4, 0, 0);
        stg.hi = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(hrs, i * 4, 0, 0);
    };
    // the dV pass reads Q by rows and dO transposed; the dK pass Q both ways and dO by rows
    auto store = [&](DkdvSlot<D> &sl) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NCH; u++) {
            const int r = crow + u * RSTEP;
            sl.q[r * (RS / 8) + ccol] = stg.q[u];
            if constexpr (DK) {
                sl.qt[r * (TS / 8) + ccol] = stg.q[u];
                sl.g[r * (RS / 8) + ccol] = stg.g[u];
            } else {
                sl.gt[r * (TS / 8) + ccol] = stg.g[u];
            }
        }
        if (tid < kDkdvStep) {
            sl.lse2[tid] = stg.lse;
            if constexpr (DK) sl.delta[tid] = stg.delta;
            sl.rlo[tid] = stg.lo;
            sl.rhi[tid] = max(stg.hi - stg.lo, 0);
        }
    };
    auto load_entry = [&](const Entry &e) __attribute__((always_inline)) {
        load(e.valid ? e.h : h_first, e.valid ? e.t : 0);
    };

    // one 32-query step on slot sl, this wavefront's keys
    auto step = [&](const DkdvSlot<D> &sl, const bool masked_flag) __attribute__((always_inline)) {
        const uint16_t *sq = (const uint16_t *)sl.q;
        // S = Q K^T (A = the query rows, B = this lane's key)
        f32x16_t s = zero16();
#pragma unroll
        for (int st = 0; st < KSTEPS; st++) {
            Frag8 a;
            a.u = *(const uint4 *)(sq + col * RS + half * 8 + st * 16);
            s = mfma32<DT>(a, bk[st], s);
            if (st % 4 == 3) __builtin_amdgcn_sched_barrier(0);  // reads at most 4 ahead
        }
        // P = exp2(S c - lse2), masked on the tiles the intervals cut; element i is query
        // 8 (i / 4) + 4 h + i % 4
        float p[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r0 = j * 8 + half * 4;
            const float4 l4 = *(const float4 *)(sl.lse2 + r0);
            const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
            int lo4[4] = {0, 0, 0, 0}, hi4[4] = {0, 0, 0, 0};
            if (masked_flag) {
                const int4 a4 = *(const int4 *)(sl.rlo + r0);
                const int4 b4 = *(const int4 *)(sl.rhi + r0);
                lo4[0] = a4.x; lo4[1] = a4.y; lo4[2] = a4.z; lo4[3] = a4.w;
                hi4[0] = b4.x; hi4[1] = b4.y; hi4[2] = b4.z; hi4[3] = b4.w;
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float x = fast_exp2(fmaf(s[4 * j + e], c2, -lv[e]));
                if (masked_flag) x = (uint32_t)(mkey - lo4[e]) < (uint32_t)hi4[e] ? x : 0.f;
                p[4 * j + e] = x;
            }
        }
        if constexpr (DK) {
            // dP = dO V^T, dS = P (dP - delta)
            const uint16_t *sg = (const uint16_t *)sl.g;
            f32x16_t dp = zero16();
#pragma unroll
            for (int st = 0; st < KSTEPS; st++) {
                Frag8 a;
                a.u = *(const uint4 *)(sg + col * RS + half * 8 + st * 16);
                dp = mfma32<DT>(a, bv[st], dp);
                if (st % 4 == 3) __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 d4 = *(const float4 *)(sl.delta + j * 8 + half * 4);
                p[4 * j + 0] *= dp[4 * j + 0] - d4.x;
                p[4 * j + 1] *= dp[4 * j + 1] - d4.y;
                p[4 * j + 2] *= dp[4 * j + 2] - d4.z;
                p[4 * j + 3] *= dp[4 * j + 3] - d4.w;
            }
        }
        // dV += P^T dO or dK += dS^T Q: A = P (dS) in the products' output layout (row = key,
        // k = query), B = dO (Q) by transposed reads of the row-major tile
        const uint16_t *sb = DK ? (const uint16_t *)sl.qt : (const uint16_t *)sl.gt;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            Frag8 pf;
            pf.u = make_uint4(pack2<DT>(p[8 * u], p[8 * u + 1]), pack2<DT>(p[8 * u + 2], p[8 * u + 3]),
                              pack2<DT>(p[8 * u + 4], p[8 * u + 5]), pack2<DT>(p[8 * u + 6], p[8 * u + 7]));
#pragma unroll
            for (int dt = 0; dt < DT32; dt++) {
                acc[dt] = mfma32<DT>(pf, lds_tr_frag(sb, TS, u * 16, dt * 32, lane), acc[dt]);
                if (dt % 4 == 3) __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    // prologue: step 0 in slot 0, step 1 loading; iteration n stores step n + 1 into the other
    // slot, loads step n + 2 and computes step n
    {
        const Entry e0 = entry(0);
        load_entry(e0);
        if (e0.valid) store(sm.slot[0]);
        load_entry(entry(1));
    }
    __syncthreads();
    // the step count up front (a counted loop keeps the accumulators in place across it): the
    // tiles whose rows see the block, once per query head of the item
    int32_t nsee = 0;
    if (j0 < Tk) {
        for (int64_t c0 = 0; c0 < ntiles; c0 += 64) {
            const int64_t tt = c0 + lane;
            const int4 r = *(const int4 *)(tr + (tt < ntiles ? tt : ntiles - 1) * 4);
            nsee += __builtin_popcountll(__ballot((tt < ntiles) & (r.x < j1) & (r.y > j0)));
        }
    }
    const int32_t nsteps = __builtin_amdgcn_readfirstlane(nsee * (hend - (int32_t)h_first));
    for (int n = 0; n < nsteps; n++) {
        const Entry e = entry(n);
        if (n + 1 < nsteps) store(sm.slot[(n + 1) & 1]);
        load_entry(entry(n + 2));
        step(sm.slot[n & 1], e.masked);
        if (wave == 0) publish(n + 4);
        __syncthreads();
    }

    // dK (scaled) or dV: lane holds column d = 32 dt + col, rows = keys 32 kw + crow(i)
    const int32_t nrows = (int32_t)(Tk - j0) - kw * 32;  // rows of this wavefront's keys in range
    const int64_t base = ((b * Tk + j0 + kw * 32) * Hkv + kh) * D + col;
    const int32_t rstride = (int32_t)(Hkv * D);
    const float f = DK ? scale : 1.f;
    if (hs == 1) {
        uint16_t *po = out + base;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = dm::crow(i, lane);
            if (r < nrows) {
#pragma unroll
                for (int dt = 0; dt < DT32; dt++)
                    po[r * rstride + dt * 32] = (uint16_t)(pack2<DT>(acc[dt][i] * f, 0.f) & 0xffffu);
            }
        }
    } else {
        const int64_t n = B * Tk * Hkv * D;
        float *po = w.kvpart + (part * 2 + (DK ? 0 : 1)) * n + base;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = dm::crow(i, lane);
            if (r < nrows) {
#pragma unroll
                for (int dt = 0; dt < DT32; dt++) po[r * rstride + dt * 32] = acc[dt][i] * f;
            }
        }
    }
}

// Both passes in one launch: work items [0, nwork) are dV passes and [nwork, 2 nwork) dK passes
// of the same (key block, key-value head, query-head part), taken in the order bwd_order makes
// over both, weighted by their products per step (32 and 48), so the dV passes fill in beside
// the longest dK passes instead of each launch ending on its own tail.
template <int DT, int D, bool PAD>
__global__ __launch_bounds__(256, 1) void bwd_dkdv_w4(MaskInfo m, int64_t B, int64_t Hq,
                                                      int64_t Hkv, float scale, AttnStrides sd,
                                                      const uint16_t *__restrict__ q,
                                                      const uint16_t *__restrict__ k,
                                                      const uint16_t *__restrict__ v,
                                                      const uint16_t *__restrict__ d_o,
                                                      const float *__restrict__ delta, BwdWs w,
                                                      uint16_t *__restrict__ dk,
                                                      uint16_t *__restrict__ dv) {
    __shared__ Dkdv4Smem<D> sm;
    const int64_t nwork = (m.tk + kKvBlock - 1) / kKvBlock * Hkv * B * w.hsplit;
    if ((int64_t)blockIdx.x >= 2 * nwork) return;
    const int64_t item = w.order[blockIdx.x];
    if (item >= nwork)
        dkdv_w4_pass<DT, D, PAD, kDkdvDK>(sm, item - nwork, m, B, Hq, Hkv, scale, sd, q, k, v, d_o,
                                          delta, w, dk);
    else
        dkdv_w4_pass<DT, D, PAD, kDkdvDV>(sm, item, m, B, Hq, Hkv, scale, sd, q, k, v, d_o, delta,
                                          w, dv);
}


void launch_dkdv_w4(int dtype, bool pad, int64_t blocks, const MaskInfo &m, int64_t B, int64_t Hq,
                    int64_t Hkv, float scale, const AttnStrides &sd, const uint16_t *q,
                    const uint16_t *k, const uint16_t *v, const uint16_t *d_o, const float *delta,
                    const BwdWs &w, uint16_t *dk, uint16_t *dv, hipStream_t st) {
#define DKDV4(DT, P)                                                                          \
    bwd_dkdv_w4<DT, 256, P><<<(unsigned)(2 * blocks), 256, 0, st>>>(m, B, Hq, Hkv, scale, sd, q, \
                                                                  k, v, d_o, delta, w, dk, dv)
    if (dtype == DM_BF16) {
        if (pad) { DKDV4(DM_BF16, true); } else { DKDV4(DM_BF16, false); }
    } else {
        if (pad) { DKDV4(DM_F16, true); } else { DKDV4(DM_F16, false); }
    }
#undef DKDV4
}

}  // namespace dm
