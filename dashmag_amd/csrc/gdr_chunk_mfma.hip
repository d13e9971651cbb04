// The chunked gated delta rule forward on gfx950 MFMA: bf16/f16 inputs, Dk and Dv multiples of 8
// up to 128 (the products are 128 wide: columns past a head width are loaded as zeros, which
// add nothing to any product or norm, keep the state's extra rows and columns at zero, and are
// never stored), f32 state
// and accumulation, the intermediates that only feed products rounded to the inputs' dtype (W, U,
// T, S, V' and Q K^T o decay, as fla's and the reference's tensor-core kernels round them,
// crates/dash-ops/src/gated_delta/chunk/cube/tc.rs:1-12).
//
//   gdr_mfma_prep    per (chunk, head), parallel: G = cumsum g; K K^T and Q K^T (MFMA); A and
//                    T = (I + A)^-1 in f32 by 16 x 16 blocks (each diagonal block by column
//                    forward substitution, the rest by block forward substitution); W = T (beta
//                    gamma K), U = T (beta V) (MFMA); Aqk = scale (Q K^T o decay) (the forward
//                    stores it transposed, with Q, as the output products' B fragments).
//   gdr_mfma_state2  per (sequence, head, 32 state columns), serial over the sequence's chunks:
//                    the state S lives in registers in the 32x32 products' output layout, which
//                    is also the operand layout of the next product, its rows split over a
//                    pair of wavefronts; V' = U - W S; S <- exp(G_last) S + (lam K)^T V'; the
//                    operands come from the prep kernel as ready-made fragments straight into
//                    registers. In the forward two more wavefronts of the workgroup form the
//                    output O^T = scale gamma (S^T Q^T) + V'^T Aqk^T from S and V' handed over
//                    in LDS; the backward's run stores S and V' as operand fragments instead.
// Notation as chunk/reference.rs:11-18 (Q scaled, G_last the chunk's last cumulative gate).
#include <mutex>
#include <string>
#include <tuple>
#include <type_traits>
#include <vector>

#include "attention_kernels.h"
#include "gdr_common.h"
#include "mfma.h"

namespace dm {

constexpr int kD = 128;         // the products' Dk = Dv (the heads' widths are at most this)
constexpr int kC = kChunk;      // 64 tokens
constexpr int kRowS = kD + 8;   // row stride read by ds_read_b128 rows
constexpr int kRowB = kD + 4;   // row stride read by ds_read_b64 rows (32 rows per half wave)
constexpr int kTrS = kD + 32;   // row stride read by ds_read_b64_tr_b16

struct MfmaWs {
    int64_t nsh;       // sequences x heads
    int32_t *seq_chunk0, *chunk_seq, *chunk_tok0, *chunk_len;
    int32_t *seq_order;  // [S]: the sequences by chunk count, the most first
    float *G;          // [ch][64]
    uint16_t *Wf;      // [ch][2 token tiles][8 dk steps][64 lanes][8]: W as A fragments of V' = W S
    uint16_t *Uc;      // [ch][4 dv tiles][2 token tiles][2][64 lanes][8]: U in the product layout
    uint16_t *Kf;      // [ch][4 dk tiles][4 token steps][64 lanes][8]: (lam K)^T as A fragments
    uint16_t *Aqk;     // [ch][64][64] row-major, scale included
    uint16_t *Sf;      // [ch][4 dv tiles][8 dk steps][64 lanes][8]: S entering the chunk
    uint16_t *Vf;      // [ch][4 dv tiles][4 token steps][64 lanes][8]: V'
    uint16_t *Qn;      // [ch][64][128] normalised queries (backward, with the l2 normalisation)
    // the forward's, instead of Aqk, Sf, Vf and Qn: what its output wavefronts load
    uint16_t *Qf;      // [ch][2 token tiles][8 dk steps][64 lanes][8]: Q (normalised) as B fragments
    uint16_t *Af;      // [ch][2 token tiles][4 key steps][64 lanes][8]: Aqk^T as B fragments
    // the backward's, besides
    uint16_t *Tm;      // [ch][64][64] T = (I + A)^-1, row-major
    uint16_t *Krf;     // [ch][2 token tiles][8 dk steps][64][8]: lam K as A fragments (rows tokens)
    uint16_t *WTf;     // [ch][4 dk tiles][4 token steps][64][8]: W^T as A fragments
    uint16_t *F;       // [ch][4 dv tiles][4 dk tiles][64][16]: (gamma Q)^T dO - W^T (Aqk^T dO)
    uint16_t *dSf;     // [ch][4 dv tiles][8 dk steps][64][8]: dS after the chunk, as S in Sf
};

static size_t mfma_layout(const dm_gdr_desc *d, char *base, MfmaWs *w, bool bwd = false) {
    const int64_t nc = gdr_chunk_bound(d), S = gdr_nseq(d), ch = nc * d->h;
    size_t off = 0;
    auto take = [&](size_t bytes) -> char * {
        char *p = base ? base + off : nullptr;
        off += align_up(bytes);
        return p;
    };
    MfmaWs x{};
    x.nsh = S * d->h;
    x.seq_chunk0 = (int32_t *)take((S + 1) * 4);
    x.chunk_seq = (int32_t *)take(nc * 4);
    x.chunk_tok0 = (int32_t *)take(nc * 4);
    x.chunk_len = (int32_t *)take(nc * 4);
    x.seq_order = (int32_t *)take(S * 4);
    x.G = (float *)take(ch * kC * 4);
    x.Wf = (uint16_t *)take(ch * kC * kD * 2);
    x.Uc = (uint16_t *)take(ch * kC * kD * 2);
    x.Kf = (uint16_t *)take(ch * kC * kD * 2);
    if (bwd) {
        x.Aqk = (uint16_t *)take(ch * kC * kC * 2);
        x.Sf = (uint16_t *)take(ch * kD * kD * 2);
        x.Vf = (uint16_t *)take(ch * kC * kD * 2);
        if (d->qk_l2norm) x.Qn = (uint16_t *)take(ch * kC * kD * 2);
    } else {
        x.Qf = (uint16_t *)take(ch * kC * kD * 2);
        x.Af = (uint16_t *)take(ch * kC * kC * 2);
    }
    if (bwd) {
        x.Tm = (uint16_t *)take(ch * kC * kC * 2);
        x.Krf = (uint16_t *)take(ch * kC * kD * 2);
        x.WTf = (uint16_t *)take(ch * kC * kD * 2);
        x.F = (uint16_t *)take(ch * kD * kD * 2);
        x.dSf = (uint16_t *)take(ch * kD * kD * 2);
    }
    if (w) *w = x;
    return off;
}

// ------------------------------------------------------------------------------------------
// Prep
// ------------------------------------------------------------------------------------------

// Unpadded 16-bit tiles of W = 128 or 64 columns with their 16-byte column chunks permuted by
// row (chunk m of row r at m ^ f(r)): the transposed fragment reads (4 rows x 64 bytes a pass of
// 32 lanes), 16-byte reads and writes of 16 consecutive rows at one column, and 16-byte row
// writes are all free of bank conflicts at 64 banks of 4 bytes; 8-byte accesses of 32 rows at one
// column are 2-way, as with padded rows. (Rows padded to 272 or 144 bytes had made every
// transposed read of the 128-column tiles a 4-way conflict and of the 64-column tiles 2-way.)
template <int W>
__device__ __forceinline__ int sw(int r, int c) {
    const int f = W == 128 ? ((r & 3) << 2) | ((r >> 2) & 3) : (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
    return r * W + ((((c >> 3) ^ f)) << 3) + (c & 7);
}
template <int W>
__device__ __forceinline__ Frag8 lds_tr_sw(const uint16_t *tile, int k0, int c0, int lane) {
    const int g = lane >> 4, i = lane & 15;
    const int row = k0 + 4 * (g >> 1) + (i >> 2);
    const int colx = c0 + 16 * (g & 1) + 4 * (i & 3);
    typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
    s16x4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(tile + sw<W>(row, colx)));
    s16x4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(tile + sw<W>(row + 8, colx)));
    Frag8 f;
    __builtin_memcpy(&f.u.x, &a, 8);
    __builtin_memcpy(&f.u.z, &b, 8);
    return f;
}
template <int W>
__device__ __forceinline__ Frag8 row_frag_sw(const uint16_t *t, int r0, int k0, int lane) {
    const int r = r0 + (lane & 31), c = k0 + (lane >> 5) * 4;
    const uint2 lo = *(const uint2 *)(t + sw<W>(r, c)), hi = *(const uint2 *)(t + sw<W>(r, c + 8));
    Frag8 f;
    f.u = make_uint4(lo.x, lo.y, hi.x, hi.y);
    return f;
}
template <int DT, int W>
__device__ __forceinline__ void store_ct_sw(uint16_t *t, int r0, int c0, const f32x16_t &v, int lane,
                                            float f = 1.f) {
    const int r = c0 + (lane & 31), c = r0 + (lane >> 5) * 4;
#pragma unroll
    for (int g = 0; g < 4; g++)
        *(uint2 *)(t + sw<W>(r, c + g * 8)) = make_uint2(pack2<DT>(v[4 * g] * f, v[4 * g + 1] * f),
                                                        pack2<DT>(v[4 * g + 2] * f, v[4 * g + 3] * f));
}
template <int DT, int W>
__device__ __forceinline__ void tile_at_out_sw(const uint16_t *t, int r0, int c0, int lane, float (&v)[16]) {
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const Frag8 f = lds_tr_sw<W>(t, r0 + 16 * hh, c0, lane);
        const uint32_t w4[4] = {f.u.x, f.u.y, f.u.z, f.u.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[8 * hh + 2 * e] = unpack_lo<DT>(w4[e]);
            v[8 * hh + 2 * e + 1] = unpack_hi<DT>(w4[e]);
        }
    }
}

// 52 KB: three workgroups per CU. The query tile's space later holds T (f32); the key tile's
// space keeps the keys until W = (T diag(beta gamma)) K, then holds beta V for U = T (beta V),
// then stages the W rows for the fragment stores. A is kept as its ten lower 16 x 16 blocks.
struct PrepSmem {
    uint4 k[kC * kRowS / 8];  // keys, rows; later beta V rows; later W rows
    uint4 q[kC * kRowS / 8];  // queries, rows; later T (f32)
    float a[10][16][20];      // A's blocks (bi, bj), bi >= bj, at bi (bi + 1) / 2 + bj; f32
    float mm[4][16][20];      // T's off-diagonal block products
    float g[kC], gam[kC], bet[kC], lam[kC];
};
static_assert(sizeof(float) * kC * (kC + 4) <= sizeof(uint4) * kC * kRowS / 8, "T in q");
static_assert(sizeof(PrepSmem) <= 160 * 1024 / 3, "three workgroups per compute unit");
// element (r, c) of A, in a lower block (r / 16 >= c / 16)
__device__ __forceinline__ float &a_at(PrepSmem &sm, int r, int c) {
    const int bi = r >> 4, bj = c >> 4;
    return sm.a[bi * (bi + 1) / 2 + bj][r & 15][c & 15];
}

template <int DT>
__global__ __launch_bounds__(256, 3) void gdr_mfma_prep(GdrArgs a, MfmaWs w) {
    __shared__ PrepSmem sm;
    const int64_t ch = blockIdx.x, n = ch / a.H, h = ch % a.H;
    const int len = w.chunk_len[n];
    if (len == 0) return;
    const int64_t tok0 = w.chunk_tok0[n];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    uint16_t *ks = (uint16_t *)sm.k, *qs = (uint16_t *)sm.q;
    float(*tt)[kC + 4] = (float(*)[kC + 4])sm.q;  // T, in the query tile's space
    float(*mm)[16][20] = sm.mm;

    // every row's loads issued before any is used (rows past the chunk's tokens read the last
    // valid row and are zeroed after); the values stay in registers until U
    uint4 vreg[4], qraw[4], kraw[4];
    {
        const uint16_t *vin = (const uint16_t *)a.v, *qin = (const uint16_t *)a.q,
                       *kin = (const uint16_t *)a.k;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int xx = tid + 256 * u, r = xx / 16, c = xx % 16;
            const int64_t tok = tok0 + (r < len ? r : len - 1);
            vreg[u] = c * 8 < a.Dv ? *(const uint4 *)(vin + v_at(a, tok, h) + c * 8) : zero4();
            qraw[u] = c * 8 < a.Dk ? *(const uint4 *)(qin + q_at(a, tok, h) + c * 8) : zero4();
            kraw[u] = c * 8 < a.Dk ? *(const uint4 *)(kin + k_at(a, tok, h) + c * 8) : zero4();
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int r = (tid + 256 * u) / 16;
            if (r >= len) vreg[u] = qraw[u] = kraw[u] = make_uint4(0, 0, 0, 0);
        }
    }
    // the gates (after the rows' loads: their reads wait on the memory counter)
    if (tid < kC) {
        const bool ok = tid < len;
        sm.g[tid] = ok ? ld_any(a.g_dt, a.g, g_at(a, tok0 + tid, h)) : 0.f;
        sm.bet[tid] = ok ? ld_any(a.beta_dt, a.beta, b_at(a, tok0 + tid, h)) : 0.f;
    }
    // queries and keys: 16 lanes per row, zero past the chunk's tokens; normalised in f32 and
    // rounded back to the dtype when asked
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int xx = tid + 256 * u, r = xx / 16, c = xx % 16;
        uint4 qv = qraw[u], kv = kraw[u];
        if (a.l2norm) {
            float qf[8], kf[8];
            const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w}, kw[4] = {kv.x, kv.y, kv.z, kv.w};
            float sq = 0.f, sk = 0.f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                qf[2 * e] = unpack_lo<DT>(qw[e]);
                qf[2 * e + 1] = unpack_hi<DT>(qw[e]);
                kf[2 * e] = unpack_lo<DT>(kw[e]);
                kf[2 * e + 1] = unpack_hi<DT>(kw[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                sq += qf[e] * qf[e];
                sk += kf[e] * kf[e];
            }
#pragma unroll
            for (int o = 8; o >= 1; o >>= 1) {
                sq += __shfl_xor(sq, o, 64);
                sk += __shfl_xor(sk, o, 64);
            }
            const float qi = 1.f / sqrtf(sq + 1e-6f), ki = 1.f / sqrtf(sk + 1e-6f);
            qv = make_uint4(pack2<DT>(qf[0] * qi, qf[1] * qi), pack2<DT>(qf[2] * qi, qf[3] * qi),
                            pack2<DT>(qf[4] * qi, qf[5] * qi), pack2<DT>(qf[6] * qi, qf[7] * qi));
            kv = make_uint4(pack2<DT>(kf[0] * ki, kf[1] * ki), pack2<DT>(kf[2] * ki, kf[3] * ki),
                            pack2<DT>(kf[4] * ki, kf[5] * ki), pack2<DT>(kf[6] * ki, kf[7] * ki));
            if (w.Qn) *(uint4 *)(w.Qn + (ch * kC + r) * kD + c * 8) = qv;
        }
        sm.q[sw<128>(r, c * 8) / 8] = qv;
        sm.k[sw<128>(r, c * 8) / 8] = kv;
    }
    __syncthreads();
    if (wave == 0) {
        // G = cumsum(g) by an inclusive scan across the wavefront (one token per lane)
        float x = sm.g[lane];
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        sm.g[lane] = x;
        sm.gam[lane] = __expf(x);
        sm.lam[lane] = __expf(__shfl(x, kC - 1, 64) - x);
        w.G[ch * kC + lane] = x;
    }
    __syncthreads();
    // (lam K)^T as the state pass's A fragments: fragment (dk tile r, token step st), lane l
    // holds dk = 32 r + l % 32 at tokens 16 st + 8 j + 4 (l / 32) + e in slot 4 j + e (the k
    // order of the V' fragments it meets): transposed reads of the key rows, then lam per token
    {
        uint16_t *kf_out = w.Kf + ch * kC * kD;
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const Frag8 kt = lds_tr_sw<128>(ks, st * 16, wave * 32, lane);
            const uint32_t kw[4] = {kt.u.x, kt.u.y, kt.u.z, kt.u.w};
            uint32_t o[4];
#pragma unroll
            for (int e2 = 0; e2 < 4; e2++) {
                // slots 2 e2, 2 e2 + 1: j = e2 / 2, e = 2 (e2 % 2) + {0, 1}
                const int tok = st * 16 + 8 * (e2 / 2) + 4 * half + 2 * (e2 % 2);
                o[e2] = pack2<DT>(unpack_lo<DT>(kw[e2]) * sm.lam[tok],
                                  unpack_hi<DT>(kw[e2]) * sm.lam[tok + 1]);
            }
            *(uint4 *)(kf_out + (size_t)((wave * 4 + st) * 64 + lane) * 8) =
                make_uint4(o[0], o[1], o[2], o[3]);
        }
        // for the backward, lam K also as A fragments with rows = tokens (the layout of W's):
        // fragment (token tile t, dk step st), lane l: row 32 t + l % 32, columns
        // 16 st + 4 (l / 32) + [0, 4) and 16 st + 8 + 4 (l / 32) + [0, 4)
        if (w.Krf) {
            uint16_t *kr_out = w.Krf + ch * kC * kD;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int f = wave * 4 + j, t = f / 8, st = f % 8, row = t * 32 + col;
                const uint2 lo4 = *(const uint2 *)(ks + sw<128>(row, st * 16 + half * 4)),
                            hi4 = *(const uint2 *)(ks + sw<128>(row, st * 16 + 8 + half * 4));
                const uint32_t kw[4] = {lo4.x, lo4.y, hi4.x, hi4.y};
                const float lm = sm.lam[row];
                uint32_t o[4];
#pragma unroll
                for (int e2 = 0; e2 < 4; e2++)
                    o[e2] = pack2<DT>(unpack_lo<DT>(kw[e2]) * lm, unpack_hi<DT>(kw[e2]) * lm);
                *(uint4 *)(kr_out + (size_t)(f * 64 + lane) * 8) = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
    }

    // K K^T and Q K^T on the lower tiles (0,0), (1,0), (1,1) (waves 0-2); A = beta (K K^T) o
    // decay strictly below the diagonal, Aqk = scale (Q K^T) o decay on and below it. Output
    // element i of tile (ti, tj): row 32 ti + 8 (i / 4) + 4 h + i % 4, column 32 tj + col.
    // The forward instead forms K Q^T o decay (key rows, query columns: Aqk^T), whose output
    // fragments are the B operands of its output products as they stand (lane = query, k =
    // key in the chain's fragment order); it also stores Q as B fragments.
    const bool fwd = w.Af != nullptr;
    uint16_t *aq_out = fwd ? nullptr : w.Aqk + ch * kC * kC;
    if (wave < 3) {
        const int ti = wave == 0 ? 0 : 1, tj = wave == 2 ? 1 : 0;
        f32x16_t kk, qk;
#pragma unroll
        for (int i = 0; i < 16; i++) kk[i] = qk[i] = 0.f;
#pragma unroll
        for (int st = 0; st < kD / 16; st++) {
            Frag8 ak, aq, bk;
            ak.u = *(const uint4 *)(ks + sw<128>(ti * 32 + col, half * 8 + st * 16));
            aq.u = *(const uint4 *)(qs + sw<128>(ti * 32 + col, half * 8 + st * 16));
            bk.u = *(const uint4 *)(ks + sw<128>(tj * 32 + col, half * 8 + st * 16));
            kk = mfma32<DT>(ak, bk, kk);
            // (A and B fragments share a layout: K(tj) rows as A and Q(ti) rows as B give
            // element (key 32 tj + crow(i), query 32 ti + col))
            qk = fwd ? mfma32<DT>(bk, aq, qk) : mfma32<DT>(aq, bk, qk);
        }
        const int j = tj * 32 + col;
        // The gates read up front (broadcast reads), then the masked exponentials without
        // branches: where the mask drops a term its exponent is zeroed (above the diagonal
        // G_i - G_j > 0) and the result selected away, so no lane waits on another's reads.
        float gr[16], br[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = ti * 32 + (i / 4) * 8 + half * 4 + (i % 4);
            gr[i] = sm.g[r];
            br[i] = sm.bet[r];
        }
        const float gj = sm.g[j];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = ti * 32 + (i / 4) * 8 + half * 4 + (i % 4);
            const bool on = r >= j;
            const float ex = __expf(on ? gr[i] - gj : 0.f);
            const float dec = on ? ex : 0.f;
            if ((r >> 4) >= (j >> 4)) a_at(sm, r, j) = r > j ? br[i] * kk[i] * dec : 0.f;
            if (!fwd) {
                const uint32_t p2 = pack2<DT>(on ? qk[i] * dec * a.scale : 0.f, 0.f);
                aq_out[r * kC + j] = (uint16_t)(p2 & 0xffffu);
            }
        }
        if (fwd) {
            // element i: key kr = 32 tj + crow(i), query qj = 32 ti + col
            const int qj = ti * 32 + col;
            float gk[16];
#pragma unroll
            for (int i = 0; i < 16; i++) gk[i] = sm.g[tj * 32 + (i / 4) * 8 + half * 4 + (i % 4)];
            const float gq = sm.g[qj];
            f32x16_t v;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int kr = tj * 32 + (i / 4) * 8 + half * 4 + (i % 4);
                const bool on = kr <= qj;
                const float ex = __expf(on ? gq - gk[i] : 0.f);
                v[i] = on ? qk[i] * ex * a.scale : 0.f;
            }
            uint16_t *af = w.Af + ch * kC * kC;
#pragma unroll
            for (int u = 0; u < 2; u++)
                *(uint4 *)(af + ((ti * 4 + 2 * tj + u) * 64 + lane) * 8) = c_frag<DT>(v, u).u;
        }
    } else if (fwd) {
        // query tile 0 sees no key of tile 1
        uint16_t *af = w.Af + ch * kC * kC;
#pragma unroll
        for (int u = 0; u < 2; u++) *(uint4 *)(af + ((2 + u) * 64 + lane) * 8) = zero4();
    } else {
        for (int xx = lane; xx < 32 * 32; xx += 64) {
            const int r = xx / 32, j = 32 + xx % 32;
            aq_out[r * kC + j] = 0;
        }
    }
    if (fwd) {
        // Q as B fragments: fragment (token tile t, dk step st), lane l: token 32 t + l % 32,
        // dk 16 st + 4 (l / 32) + [0, 4) and 16 st + 8 + 4 (l / 32) + [0, 4); four a wavefront
        uint16_t *qf = w.Qf + ch * kC * kD;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int f = wave * 4 + i, t = f / 8, st = f % 8;
            const uint2 lo = *(const uint2 *)(qs + sw<128>(t * 32 + col, st * 16 + half * 4)),
                        hi = *(const uint2 *)(qs + sw<128>(t * 32 + col, st * 16 + 8 + half * 4));
            *(uint4 *)(qf + (f * 64 + lane) * 8) = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
    }
    __syncthreads();  // the query tile is dead from here; the key tile lives until W

    // T = (I + A)^-1 by 16 x 16 blocks. Diagonal block b (wave b), row by row, lane c holding
    // column c in registers: T[i][c] = [i == c] - sum_{x < i} A[i][x] T[x][c] (rows of A read
    // as broadcasts; T[x][c] = 0 for x < c makes the sum start at c).
    {
        const int b = wave, c = lane & 15;
        float tc[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            // four partial sums (by x mod 4), so a row waits on about i / 4 dependent products
            float sp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int x4 = 0; x4 < i; x4 += 4) {
                const float4 a4 = *(const float4 *)&a_at(sm, 16 * b + i, 16 * b + x4);
                const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (x4 + e < i) sp[e] += av[e] * tc[x4 + e];
            }
            tc[i] = (i == c ? 1.f : 0.f) - ((sp[0] + sp[1]) + (sp[2] + sp[3]));
        }
        if (lane < 16) {
#pragma unroll
            for (int i = 0; i < 16; i++) tt[16 * b + i][16 * b + c] = tc[i];
        }
        // the strictly upper blocks of T are zero
        for (int xx = lane; xx < 256; xx += 64) {
            const int r = xx / 16, cc = xx % 16;
            for (int bj = b + 1; bj < 4; bj++) tt[16 * b + r][16 * bj + cc] = 0.f;
        }
    }
    __syncthreads();
    // Off-diagonal blocks by doubling (T of a block-lower-triangular matrix from its diagonal
    // blocks' inverses). Step 1, the 32 x 32 diagonal halves: waves 0 and 1 form
    // M = A_{b+1,b} T_bb, then T_{b+1,b} = -T_{b+1,b+1} M (b = 0, 2). Step 2, the lower-left 32 x 32
    // quarter: wave w forms block (i, j) = (2 + w / 2, w % 2) of X = A[2:4, 0:2] T[0:2, 0:2],
    // then of T[2:4, 0:2] = -T[2:4, 2:4] X. Lane: column cc = lane % 16, rows 4 (lane / 16) + e.
    {
        const int cc = lane & 15, r0 = 4 * (lane >> 4);
        // acc[e] += sum_y A(16 bi + r0 + e, 16 kb + y) T(16 kb + y, 16 bj + cc)
        auto a_times_t = [&](float (&acc)[4], int bi, int kb, int bj) {
            float tcol[16];
#pragma unroll
            for (int y = 0; y < 16; y++) tcol[y] = tt[16 * kb + y][16 * bj + cc];
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int y4 = 0; y4 < 16; y4 += 4) {
                    const float4 a4 = *(const float4 *)&a_at(sm, 16 * bi + r0 + e, 16 * kb + y4);
                    acc[e] += a4.x * tcol[y4] + a4.y * tcol[y4 + 1] + a4.z * tcol[y4 + 2] +
                              a4.w * tcol[y4 + 3];
                }
        };
        // acc[e] += sum_y T(16 bi + r0 + e, 16 kb + y) X_m(y, cc)
        auto t_times_m = [&](float (&acc)[4], int bi, int kb, int m) {
            float mcol[16];
#pragma unroll
            for (int y = 0; y < 16; y++) mcol[y] = mm[m][y][cc];
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int y4 = 0; y4 < 16; y4 += 4) {
                    const float4 t4 = *(const float4 *)&tt[16 * bi + r0 + e][16 * kb + y4];
                    acc[e] += t4.x * mcol[y4] + t4.y * mcol[y4 + 1] + t4.z * mcol[y4 + 2] +
                              t4.w * mcol[y4 + 3];
                }
        };
        if (wave < 2) {
            const int bj = 2 * wave, bi = bj + 1;
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            a_times_t(acc, bi, bj, bj);
#pragma unroll
            for (int e = 0; e < 4; e++) mm[wave][r0 + e][cc] = acc[e];
        }
        __syncthreads();
        if (wave < 2) {
            const int bj = 2 * wave, bi = bj + 1;
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            t_times_m(acc, bi, bi, wave);
#pragma unroll
            for (int e = 0; e < 4; e++) tt[16 * bi + r0 + e][16 * bj + cc] = -acc[e];
        }
        __syncthreads();
        const int bi = 2 + (wave >> 1), bj = wave & 1;
        {
            // X_{bi,bj} = sum over k = bj .. 1 of A_{bi,k} T_{k,bj} (T_{0,1} = 0)
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            for (int kb = bj; kb < 2; kb++) a_times_t(acc, bi, kb, bj);
#pragma unroll
            for (int e = 0; e < 4; e++) mm[wave][r0 + e][cc] = acc[e];
        }
        __syncthreads();
        {
            // T_{bi,bj} = -(sum over k = 2 .. bi of T_{bi,k} X_{k,bj}); X_{k,bj} is wave 2 (k - 2) + bj's
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            for (int kb = 2; kb <= bi; kb++) t_times_m(acc, bi, kb, 2 * (kb - 2) + bj);
#pragma unroll
            for (int e = 0; e < 4; e++) tt[16 * bi + r0 + e][16 * bj + cc] = -acc[e];
        }
        __syncthreads();
    }

    // W = (T diag(beta gamma)) K, then U = T (beta V): 8 output tiles each (2 token rows x 4
    // columns of 32), wave w taking column tile w. A = T rows (f32 -> dtype; for W each column
    // scaled by its token's beta gamma) with k slots 16 st + 8 j + 4 h + e, B = the key rows,
    // then the beta V rows, read transposed (k = token, col = column).
    f32x16_t wt[2], ut[2];
    auto tfrag = [&](int ti, int st, bool bg) __attribute__((always_inline)) {
        const int c0 = st * 16 + half * 4;
        const float *tr = &tt[ti * 32 + col][c0];
        float f[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
        if (bg) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                f[e] = sm.bet[c0 + e] * sm.gam[c0 + e];
                f[4 + e] = sm.bet[c0 + 8 + e] * sm.gam[c0 + 8 + e];
            }
        }
        Frag8 at;
        at.u = make_uint4(pack2<DT>(tr[0] * f[0], tr[1] * f[1]), pack2<DT>(tr[2] * f[2], tr[3] * f[3]),
                          pack2<DT>(tr[8] * f[4], tr[9] * f[5]), pack2<DT>(tr[10] * f[6], tr[11] * f[7]));
        return at;
    };
#pragma unroll
    for (int ti = 0; ti < 2; ti++) {
        wt[ti] = zero16();
#pragma unroll
        for (int st = 0; st < kC / 16; st++)
            wt[ti] = mfma32<DT>(tfrag(ti, st, true), lds_tr_sw<128>(ks, st * 16, wave * 32, lane), wt[ti]);
    }
    __syncthreads();  // the key tile is dead from here
    // beta V rows for U's product, in the key tile's space
    uint16_t *vs = ks;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int xx = tid + 256 * u, r = xx / 16, c = xx % 16;
        const float fv = sm.bet[r];
        const uint32_t vw[4] = {vreg[u].x, vreg[u].y, vreg[u].z, vreg[u].w};
        uint32_t vo[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            vo[e] = pack2<DT>(unpack_lo<DT>(vw[e]) * fv, unpack_hi<DT>(vw[e]) * fv);
        *(uint4 *)(vs + sw<128>(r, c * 8)) = make_uint4(vo[0], vo[1], vo[2], vo[3]);
    }
    __syncthreads();
#pragma unroll
    for (int ti = 0; ti < 2; ti++) {
        ut[ti] = zero16();
#pragma unroll
        for (int st = 0; st < kC / 16; st++)
            ut[ti] = mfma32<DT>(tfrag(ti, st, false), lds_tr_sw<128>(vs, st * 16, wave * 32, lane), ut[ti]);
    }
    __syncthreads();
    // for the backward: T, row-major in the dtype
    if (w.Tm) {
        uint16_t *tout = w.Tm + ch * kC * kC;
        for (int xx = tid; xx < kC * kC / 2; xx += 256) {
            const int r = xx / (kC / 2), c2 = (xx % (kC / 2)) * 2;
            *(uint32_t *)(tout + r * kC + c2) = pack2<DT>(tt[r][c2], tt[r][c2 + 1]);
        }
    }
    // U in the state pass's layout: that of the products' output, the lane's 16 values of
    // token tile ti as two 16-byte pieces
    {
        uint16_t *uc = w.Uc + ch * kC * kD + (size_t)wave * 2 * 2 * 64 * 8;
#pragma unroll
        for (int ti = 0; ti < 2; ti++)
#pragma unroll
            for (int qq = 0; qq < 2; qq++) {
                *(uint4 *)(uc + ((ti * 2 + qq) * 64 + lane) * 8) =
                    make_uint4(pack2<DT>(ut[ti][8 * qq + 0], ut[ti][8 * qq + 1]),
                               pack2<DT>(ut[ti][8 * qq + 2], ut[ti][8 * qq + 3]),
                               pack2<DT>(ut[ti][8 * qq + 4], ut[ti][8 * qq + 5]),
                               pack2<DT>(ut[ti][8 * qq + 6], ut[ti][8 * qq + 7]));
            }
    }
    // W as the state pass's A fragments: stage the rows (element i: row 32 ti + 8 (i / 4) +
    // 4 h + i % 4, column 32 wave + col), then fragment (token tile t, dk step st), lane l:
    // row 32 t + l % 32, columns 16 st + 4 (l / 32) + [0, 4) and 16 st + 8 + 4 (l / 32) + [0, 4)
    {
        uint16_t *wrows = (uint16_t *)sm.k;
#pragma unroll
        for (int ti = 0; ti < 2; ti++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int r = ti * 32 + (i / 4) * 8 + half * 4 + (i % 4);
                wrows[sw<128>(r, wave * 32 + col)] = (uint16_t)(pack2<DT>(wt[ti][i], 0.f) & 0xffffu);
            }
        __syncthreads();
        uint16_t *wf = w.Wf + ch * kC * kD;
        for (int xx = tid; xx < 16 * 64; xx += 256) {
            const int f = xx / 64, l = xx % 64, t = f / 8, st = f % 8;
            const int wr = t * 32 + (l & 31), wc = st * 16 + (l >> 5) * 4;
            const uint2 lo4 = *(const uint2 *)(wrows + sw<128>(wr, wc)),
                        hi4 = *(const uint2 *)(wrows + sw<128>(wr, wc + 8));
            *(uint4 *)(wf + (size_t)xx * 8) = make_uint4(lo4.x, lo4.y, hi4.x, hi4.y);
        }
        // for the backward, W^T as A fragments (rows dk, k = tokens), as (lam K)^T in Kf
        if (w.WTf) {
            uint16_t *wt_out = w.WTf + ch * kC * kD;
#pragma unroll
            for (int st = 0; st < 4; st++) {
                const Frag8 x = lds_tr_sw<128>(wrows, st * 16, wave * 32, lane);
                *(uint4 *)(wt_out + (size_t)((wave * 4 + st) * 64 + lane) * 8) = x.u;
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// State pass
// ------------------------------------------------------------------------------------------

// The state passes' workgroup -> (sequence x head, column block): workgroup x goes to XCD x % 8,
// and the four column blocks of a (sequence, head) take workgroups 8 apart, so they share one
// XCD's L2 (the operands are read from HBM once). The (sequence, head) items are taken in the
// plan's sequence order, the longest chains first, so they are dispatched first. Grid:
// state_grid(nsh) workgroups.
__host__ __device__ inline int64_t state_grid(int64_t nsh) { return (nsh + 7) / 8 * 32; }
__device__ __forceinline__ bool state_item(int64_t x, int64_t nsh, const int32_t *order,
                                           int64_t H, int64_t *sh, int *wave) {
    const int64_t xcd = x % 8, y = x / 8;
    *wave = (int)(y % 4);
    const int64_t idx = (y / 4) * 8 + xcd;
    if (idx >= nsh) return false;
    *sh = (int64_t)order[idx / H] * H + idx % H;
    return true;
}

// The state pass with the rows of S split over a pair of wavefronts (one workgroup per column
// block): wavefront p holds rows 64 p + [0, 64) of the block's 32 columns. Per chunk each
// computes its part of W S (8 products over its 64 state rows), the pair swaps the parts through
// LDS (two buffers by chunk parity: one barrier per chunk), both form V' = U - W S, and each
// updates its own rows: S_p <- e^{G_last} S_p + (lam K)_p^T V' (8 products). Per wavefront
// that is half the products, half the operands and half the state of a single wavefront per
// block, on the chain every chunk waits for.
constexpr int kStateParts = 2;  // wavefronts sharing a column block's state rows (4 measured slower)

#ifdef DM_TRACE_STATE
// profiling aid (built only with -DDM_TRACE_STATE=<sequence x head>): per-chunk clock stamps of
// wavefront 0 of that item's first column block, and the 100 MHz clock at its start and end
__device__ uint64_t dm_trace_state[256][6];
__device__ uint64_t dm_trace_out[256][6];
#define DM_SSTAMP(c, k)                                                                          \
    do {                                                                                        \
        if (sh == (DM_TRACE_STATE) && blk == 0 && p == 0 && lane == 0 && (c) - c0 < 254)        \
            dm_trace_state[(c) - c0][k] = __builtin_readcyclecounter();                         \
    } while (0)
#define DM_OSTAMP(c, k)                                                                          \
    do {                                                                                        \
        if (traced && t == 0 && lane == 0 && (c) - c0 < 254)                                    \
            dm_trace_out[(c) - c0][k] = __builtin_readcyclecounter();                           \
    } while (0)
#else
#define DM_SSTAMP(c, k) \
    do {                \
    } while (0)
#define DM_OSTAMP(c, k) \
    do {                \
    } while (0)
#endif

template <int NP>
struct PartOps {
    static constexpr int RT = 4 / NP, KS = 8 / NP;  // state tiles and dk steps per wavefront
    Frag8 wf[2][KS];  // W: token tile t, dk step KS p + st
    Frag8 uc[2];      // U: token tile t, the 8-value half p of the lane's 16 (NP = 2)
    Frag8 kf[RT][4];  // (lam K)^T: dk tile RT p + r, token step st
    float glast;
};

// OUT: the workgroup also computes the chunks' outputs, on two more wavefronts (one per token
// tile, on SIMDs the chain leaves idle): the chain hands each chunk's S and V' over in LDS
// instead of storing them, and the output wavefronts form O^T = scale gamma (S^T Q^T) +
// V'^T Aqk^T for the block's 32 columns one chunk behind, in the barriers' rhythm.
// The output wavefronts of the fused state pass: token tile t of each chunk, the block's 32
// columns. Q^T and Aqk^T come as the B fragments the prep kernel stored (lane = token, k slots
// 16 st + 8 (j / 4) + 4 (l / 32) + j % 4, the order of the chain's fragments), loaded two
// chunks ahead; S^T and V'^T are the chain's fragments as A operands.
constexpr int kOutRow = 40;  // 16-bit elements a row of an output tile in LDS (32 + 8)
struct OutOps {
    Frag8 q[8], aq[4];
    float gam;
    int len;
    int64_t tok0;
};
template <int DT, int NP, int KS>
__device__ __forceinline__ void state_output(const GdrArgs &a, const MfmaWs &w, void *out,
                                             const uint4 (*sbuf)[NP][KS][64],
                                             const uint4 (*vbuf)[4][64], uint16_t *otiles,
                                             int64_t h, int blk, int c0, int c1, int t, int lane,
                                             bool traced) {
    const int col = lane & 31, half = lane >> 5;
    const int r = t * 32 + col;  // this lane's token within the chunk (column of O^T)
    // the sequence's tokens, read once: chunk c starts 64 (c - c0) tokens into them (no load
    // in the chunk loop waits on another)
    int64_t first = 0, end = 0;
    if (c0 < c1) {
        first = w.chunk_tok0[c0];
        end = (int64_t)w.chunk_tok0[c1 - 1] + w.chunk_len[c1 - 1];
    }
    // the block's output columns blk * 32 + [0, 32) of the rows
    uint16_t *obase0 = (uint16_t *)out + h * a.Dv + blk * 32;
    const int64_t orow_stride = a.H * a.Dv;
    const int ocols0 = (int)a.Dv - blk * 32;  // columns of the block within the head
    uint16_t *otile = otiles + t * 32 * kOutRow;
    auto load = [&](int c, OutOps &x) __attribute__((always_inline)) {
        c = c < c1 ? c : c1 - 1;
        const int64_t ch = (int64_t)c * a.H + h;
        const int64_t tok0 = first + (int64_t)(c - c0) * kC;
        const uint16_t *qf = w.Qf + ch * kC * kD + (size_t)t * 8 * 64 * 8 + lane * 8;
        const uint16_t *af = w.Af + ch * kC * kC + (size_t)t * 4 * 64 * 8 + lane * 8;
#pragma unroll
        for (int st = 0; st < 8; st++) x.q[st].u = *(const uint4 *)(qf + st * 64 * 8);
#pragma unroll
        for (int st = 0; st < 4; st++) x.aq[st].u = *(const uint4 *)(af + st * 64 * 8);
        x.gam = w.G[ch * kC + r];
        x.len = (int)(end - tok0 < kC ? end - tok0 : kC);
        x.tok0 = tok0;
    };
    auto emit = [&](int c, const OutOps &x) __attribute__((always_inline)) {
        DM_OSTAMP(c, 0);
        Frag8 sa[8], va[4];
#pragma unroll
        for (int st = 0; st < 8; st++) sa[st].u = sbuf[c % 3][st / KS][st % KS][lane];
#pragma unroll
        for (int st = 0; st < 4; st++) va[st].u = vbuf[c & 1][st][lane];
        DM_OSTAMP(c, 1);
        f32x16_t inter = zero16(), intra = zero16();
#pragma unroll
        for (int st = 0; st < 8; st++) {
            inter = mfma32<DT>(sa[st], x.q[st], inter);
            if (st < 4) intra = mfma32<DT>(va[st], x.aq[st], intra);
        }
        DM_OSTAMP(c, 2);
        const float f = a.scale * __expf(x.gam);
        // the tile through LDS, token rows of the block's 32 columns: lane (token r) writes its
        // 16 values as 8-byte pieces, then each lane stores 16 bytes of a row (4 lanes a row, 16
        // rows an instruction). 8-byte stores straight from the products' layout touched 32 rows
        // an instruction, and cost the pass about 45 us on config 4 (316 -> 272 us).
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++)
            *(uint2 *)(otile + col * kOutRow + g4 * 8 + half * 4) = make_uint2(
                pack2<DT>(inter[4 * g4] * f + intra[4 * g4], inter[4 * g4 + 1] * f + intra[4 * g4 + 1]),
                pack2<DT>(inter[4 * g4 + 2] * f + intra[4 * g4 + 2], inter[4 * g4 + 3] * f + intra[4 * g4 + 3]));
        __builtin_amdgcn_wave_barrier();  // (a wavefront's LDS accesses complete in order)
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int rr = k * 16 + (lane >> 2), piece = lane & 3;
            const uint4 v = *(const uint4 *)(otile + rr * kOutRow + piece * 8);
            if (t * 32 + rr < x.len && piece * 8 < ocols0)
                *(uint4 *)(obase0 + (x.tok0 + t * 32 + rr) * orow_stride + piece * 8) = v;
        }
        __builtin_amdgcn_wave_barrier();
        DM_OSTAMP(c, 3);
    };
    // one barrier per chunk of the chain plus its last one; after barrier b the chunk b - 1
    // has its S and V' in LDS
    OutOps oa, ob;
    if (c0 < c1) {
        load(c0, oa);
        load(c0 + 1, ob);
    }
    __syncthreads();  // barrier c0
    int b = c0 + 1;
    for (; b + 1 <= c1; b += 2) {
        __syncthreads();  // barrier b
        emit(b - 1, oa);
        load(b + 1, oa);
        DM_OSTAMP(b - 1, 4);
        __syncthreads();  // barrier b + 1
        emit(b, ob);
        load(b + 2, ob);
        DM_OSTAMP(b, 4);
    }
    if (b <= c1) {
        __syncthreads();
        emit(b - 1, oa);
    }
}

template <int DT, int NP, bool OUT>
__global__ __launch_bounds__(64 * NP + (OUT ? 128 : 0), 1) void gdr_mfma_state2(
    GdrArgs a, MfmaWs w, const float *h0, float *final_state, void *out) {
    constexpr int RT = 4 / NP, KS = 8 / NP;
    static_assert(NP == 2, "U's rows are split over two wavefronts");
    using HalfOps = PartOps<NP>;
    __shared__ __align__(16) float4 xch[2][NP][2][4][64];  // [parity][wavefront][token tile][i / 4][lane]
    // OUT: S by chunk mod 3 (written before a step's barrier, read after the next one, while
    // the chain writes the chunk after next) and V' by chunk parity (written after a step's
    // barrier), both as the fragments the chain formed
    __shared__ __align__(16) uint4 sbuf[OUT ? 3 : 1][NP][KS][64];
    __shared__ __align__(16) uint4 vbuf[OUT ? 2 : 1][4][64];
    // OUT: an output tile (32 tokens x 32 columns) a output wavefront, for its stores
    __shared__ __align__(16) uint16_t otiles[OUT ? 2 * 32 * kOutRow : 8];
    int64_t sh;
    int blk;
    if (!state_item(blockIdx.x, w.nsh, w.seq_order, a.H, &sh, &blk)) return;
    const int64_t s = sh / a.H, h = sh % a.H;
    const int lane = threadIdx.x & 63;
    const int p = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // row part (>= NP: output)
    const int col = lane & 31;
    const int c0 = w.seq_chunk0[s], c1 = w.seq_chunk0[s + 1];
    const int dv = blk * 32 + col;
    if (OUT && p >= NP) {
#ifdef DM_TRACE_STATE
        const bool traced = sh == (DM_TRACE_STATE) && blk == 0;
#else
        const bool traced = false;
#endif
        state_output<DT, NP, KS>(a, w, out, sbuf, vbuf, otiles, h, blk, c0, c1, p - NP, lane,
                                 traced);
        return;
    }

    // S_p: tile r holds rows 32 (RT p + r) + crow(i) of column dv
    f32x16_t S[RT];
    {
        const float *src = h0 ? h0 + sh * a.Dk * a.Dv : nullptr;
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int row = (RT * p + r) * 32 + crow(i, lane);
                S[r][i] = src && row < a.Dk && dv < a.Dv ? src[row * a.Dv + dv] : 0.f;
            }
    }
    // -I's rows 16 p + [0, 16) as the A operand against U's half p as the B operand: lane l's B
    // slot j is token row crow(8 p + j, l) = 16 p + 8 (j / 4) + 4 (l / 32) + j % 4 at hardware
    // k = 8 (l / 32) + j, so A(row, k) = -1 exactly where that row is the lane's row l % 32.
    Frag8 negid;
    {
        const uint16_t m1 = DT == DM_BF16 ? 0xBF80 : 0xBC00;  // -1 in bf16 / f16
        uint16_t e[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            e[j] = (lane & 31) == 16 * p + 8 * (j / 4) + 4 * (lane >> 5) + (j % 4) ? m1 : 0;
        negid.u = make_uint4(e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16,
                             e[4] | (uint32_t)e[5] << 16, e[6] | (uint32_t)e[7] << 16);
    }
    // a chunk's operands in two parts: W and U (free once W S is issued) and (lam K)^T with
    // G_last (free once the update is issued)
    auto load_wu = [&](int c, HalfOps &x) __attribute__((always_inline)) {
        c = c < c1 ? c : c1 - 1;
        const int64_t ch = (int64_t)c * a.H + h;
        const uint16_t *wf = w.Wf + ch * kC * kD;
        const uint16_t *uc = w.Uc + ch * kC * kD + (size_t)blk * 2 * 2 * 64 * 8;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int st = 0; st < KS; st++)
                x.wf[t][st].u = *(const uint4 *)(wf + ((t * 8 + p * KS + st) * 64 + lane) * 8);
#pragma unroll
        for (int t = 0; t < 2; t++) x.uc[t].u = *(const uint4 *)(uc + ((t * 2 + p) * 64 + lane) * 8);
    };
    auto load_k = [&](int c, HalfOps &x) __attribute__((always_inline)) {
        c = c < c1 ? c : c1 - 1;
        const int64_t ch = (int64_t)c * a.H + h;
        const uint16_t *kf = w.Kf + ch * kC * kD;
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int st = 0; st < 4; st++)
                x.kf[r][st].u = *(const uint4 *)(kf + (((p * RT + r) * 4 + st) * 64 + lane) * 8);
        x.glast = w.G[ch * kC + kC - 1];
    };
    // chunk c's step on the operands in x, which then load chunk cn's (each part as soon as the
    // step's products have taken it, so the loads issue while the products run)
    auto step = [&](int c, HalfOps &x, int cn) __attribute__((always_inline)) {
        const int64_t ch = (int64_t)c * a.H + h;
        DM_SSTAMP(c, 0);
        // this part of S as operand fragments (dk steps KS p + st), also stored for the output
        Frag8 sf[KS];
        uint16_t *sfo = w.Sf + ch * kD * kD + (size_t)blk * 8 * 64 * 8;
#pragma unroll
        for (int st = 0; st < KS; st++) {
            sf[st] = c_frag<DT>(S[st / 2], st % 2);
            if (OUT)
                sbuf[OUT ? c % 3 : 0][p][st][lane] = sf[st].u;
            else
                *(uint4 *)(sfo + ((p * KS + st) * 64 + lane) * 8) = sf[st].u;
        }
        // this part's share of W S - U: the products start from -U's rows 16 p + [0, 16) of each
        // token tile (U as a B operand times -I, exact in f32), so the pair's sum is W S - U
        f32x16_t vp[2];
#pragma unroll
        for (int t = 0; t < 2; t++) vp[t] = mfma32<DT>(negid, x.uc[t], zero16());
#pragma unroll
        for (int st = 0; st < KS; st++)
#pragma unroll
            for (int t = 0; t < 2; t++) vp[t] = mfma32<DT>(x.wf[t][st], sf[st], vp[t]);
        // the decay of this part of S, on the vector unit while the products run
        const float gl = __expf(x.glast);
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int i = 0; i < 16; i++) S[r][i] *= gl;
        load_wu(cn, x);
        // swap the shares: each wavefront reads the other's (x + y = y + x exactly, so both
        // wavefronts form the same V')
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                xch[c & 1][p][t][g][lane] =
                    make_float4(vp[t][4 * g], vp[t][4 * g + 1], vp[t][4 * g + 2], vp[t][4 * g + 3]);
        DM_SSTAMP(c, 1);
        __syncthreads();
        DM_SSTAMP(c, 2);
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                // V' = -(W S - U) = -(own part) - (other part)
                const float4 y = xch[c & 1][p ^ 1][t][g][lane];
                vp[t][4 * g] = -vp[t][4 * g] - y.x;
                vp[t][4 * g + 1] = -vp[t][4 * g + 1] - y.y;
                vp[t][4 * g + 2] = -vp[t][4 * g + 2] - y.z;
                vp[t][4 * g + 3] = -vp[t][4 * g + 3] - y.w;
            }
        // V' (the same in every wavefront; wavefront p stores the steps st = p mod NP)
        Frag8 vlf[4];
        uint16_t *vfo = w.Vf ? w.Vf + ch * kC * kD + (size_t)blk * 4 * 64 * 8 : nullptr;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int st = t * 2 + u;
                vlf[st] = c_frag<DT>(vp[t], u);
                if (st % NP == p) {
                    if (OUT)
                        vbuf[c & 1][st][lane] = vlf[st].u;
                    else if (vfo)
                        *(uint4 *)(vfo + (st * 64 + lane) * 8) = vlf[st].u;
                }
            }
        DM_SSTAMP(c, 3);
        // S_p <- exp(G_last) S_p + (lam K)_p^T V' (the decay applied above)
#pragma unroll
        for (int st = 0; st < 4; st++)
#pragma unroll
            for (int r = 0; r < RT; r++) S[r] = mfma32<DT>(x.kf[r][st], vlf[st], S[r]);
        load_k(cn, x);
        DM_SSTAMP(c, 4);
    };
#ifdef DM_TRACE_STATE
    if (sh == (DM_TRACE_STATE) && blk == 0 && p == 0 && lane == 0) {
        dm_trace_state[255][0] = __builtin_readcyclecounter();
        dm_trace_state[255][1] = __builtin_amdgcn_s_memrealtime();
    }
#endif
    HalfOps oa, ob;
    if (c0 < c1) {
        load_wu(c0, oa);
        load_k(c0, oa);
        load_wu(c0 + 1, ob);
        load_k(c0 + 1, ob);
    }
    // two chunks a pass, each register set loading the chunk two ahead; an odd last chunk after
    // the loop (every pass through the loop then issues the same loads, so the compiler's wait
    // counts keep the next chunks' loads in flight across a step)
    int c = c0;
    for (; c + 1 < c1; c += 2) {
        step(c, oa, c + 2);
        step(c + 1, ob, c + 3);
    }
    if (c < c1) step(c, oa, c + 2);
    if (OUT) __syncthreads();  // the last chunk's V' to the output wavefronts
#ifdef DM_TRACE_STATE
    if (sh == (DM_TRACE_STATE) && blk == 0 && p == 0 && lane == 0) {
        dm_trace_state[254][0] = __builtin_readcyclecounter();
        dm_trace_state[254][1] = __builtin_amdgcn_s_memrealtime();
    }
#endif
    if (final_state) {
        float *dst = final_state + sh * a.Dk * a.Dv;
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int row = (RT * p + r) * 32 + crow(i, lane);
                if (row < a.Dk && dv < a.Dv) dst[row * a.Dv + dv] = S[r][i];
            }
    }
}

// ------------------------------------------------------------------------------------------
// Backward (chunk/reference.rs:519-695 restated for the products; notation as the forward's)
// ------------------------------------------------------------------------------------------
//
//   gdr_bwd_pre    per (chunk, head): F = (gamma scale Q)^T dO - W^T (Aqk^T dO), the part of
//                  the state gradient's chunk step that does not depend on the state
//   gdr_bwd_state2 per (sequence, head, 32 state columns), serial over the chunks in reverse:
//                  dS_c = exp(G_last) dS_{c+1} - W^T ((lam K) dS_{c+1}) + F; stores dS_{c+1}
//                  per chunk and dh0
//   gdr_bwd_grads  per (chunk, head): dV' = (lam K) dS_{c+1} + Aqk^T dO, then every gradient
//                  the chunk gives (dq, dk, dv, dg, dbeta)

// Its 16 values stored transposed into a row-major 16-bit tile X^T: row (the tile's column)
// c0 + lane % 32, columns r0 + crow(i): runs of 4, 8-byte stores.
template <int DT>
__device__ __forceinline__ void store_ct(uint16_t *t, int stride, int r0, int c0,
                                         const f32x16_t &v, int lane, float f = 1.f) {
    uint16_t *row = t + (c0 + (lane & 31)) * stride + r0 + (lane >> 5) * 4;
#pragma unroll
    for (int g = 0; g < 4; g++)
        *(uint2 *)(row + g * 8) = make_uint2(pack2<DT>(v[4 * g] * f, v[4 * g + 1] * f),
                                             pack2<DT>(v[4 * g + 2] * f, v[4 * g + 3] * f));
}

// Sum over the 32 lanes that share lane / 32 (the columns of a product tile).
__device__ __forceinline__ float sum32(float x) { return group_sum<32>(x); }

// Row sums of a 32x32 product tile held as its output fragment (v[i]: row crow(i, lane), column
// lane % 32), by a reduce-scatter over the 32 lanes of each half: at each stage a lane keeps half
// of its values and adds its partner's copy of them, the partners pairing by lane bit 4 (a
// swizzle), 3 (row_ror 8), 2 (row_half_mirror), 1 and 0 (quad swaps), each pairing lanes that
// agree on the bits already used. Lane l ends with the sum of value 8 b4 + 4 b3 + 2 b2 + b1
// (b_k = bit k of l), as do lanes l ^ 1; returns it and that value's row in *row. 31 moves and
// adds in place of 16 reductions of 5 each.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float tile_rowsum(const float (&v)[16], int lane, int *row) {
    const bool b4 = lane & 16, b3 = lane & 8, b2 = lane & 4, b1 = lane & 2;
    float a8[8], a4[4], a2[2];
#pragma unroll
    for (int k = 0; k < 8; k++)
        a8[k] = (b4 ? v[8 + k] : v[k]) + __shfl_xor(b4 ? v[k] : v[8 + k], 16, 64);
#pragma unroll
    for (int k = 0; k < 4; k++)
        a4[k] = (b3 ? a8[4 + k] : a8[k]) + dpp_f<0x128>(b3 ? a8[k] : a8[4 + k]);  // row_ror:8
#pragma unroll
    for (int k = 0; k < 2; k++)
        a2[k] = (b2 ? a4[2 + k] : a4[k]) + dpp_f<0x141>(b2 ? a4[k] : a4[2 + k]);  // half mirror
    const float a1 = (b1 ? a2[1] : a2[0]) + dpp_f<0x4E>(b1 ? a2[0] : a2[1]);  // quad [2,3,0,1]
    *row = crow(8 * b4 + 4 * b3 + 2 * b2 + b1, lane);
    return a1 + dpp_f<0xB1>(a1);  // quad [1,0,3,2]
}

constexpr int kR = kD + 8;  // 128-column tiles (row and transposed reads)
constexpr int kT = kC + 8;  // 64-column tiles

// F per (chunk, head): wave w takes state columns 32 w + [0, 32).
struct BwdPreSmem {
    uint16_t dO[kC * kR];   // dO rows
    uint16_t qg[kC * kR];   // gamma scale Q rows
    uint16_t aq[kC * kT];   // Aqk rows
};

template <int DT>
__global__ __launch_bounds__(256) void gdr_bwd_pre(GdrArgs a, MfmaWs w, const void *d_out) {
    __shared__ BwdPreSmem sm;
    const int64_t ch = blockIdx.x, n = ch / a.H, h = ch % a.H;
    const int len = w.chunk_len[n];
    if (len == 0) return;
    const int64_t tok0 = w.chunk_tok0[n];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint16_t *dob = (const uint16_t *)d_out, *qin = (const uint16_t *)a.q;
    // every load issued first: the rows, Aqk, the gates, and W^T's fragments
    uint4 dv[4], qv[4], av[2];
    float gv[4];
    Frag8 wa[4][4];
    {
        const uint16_t *wtf = w.WTf + ch * kC * kD;
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int st = 0; st < 4; st++)
                wa[r][st].u = *(const uint4 *)(wtf + ((r * 4 + st) * 64 + lane) * 8);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) gv[u] = w.G[ch * kC + (tid + 256 * u) / 16];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int x = tid + 256 * u, r = x / 16, c = x % 16;
        const int64_t tok = tok0 + (r < len ? r : len - 1);
        dv[u] = c * 8 < a.Dv ? *(const uint4 *)(dob + o_at(a, tok, h) + c * 8) : zero4();
        qv[u] = a.l2norm      ? *(const uint4 *)(w.Qn + (ch * kC + r) * kD + c * 8)
                : c * 8 < a.Dk ? *(const uint4 *)(qin + q_at(a, tok, h) + c * 8)
                               : zero4();
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int x = tid + 256 * u, r = x / 8, c = x % 8;
        av[u] = *(const uint4 *)(w.Aqk + ch * kC * kC + r * kC + c * 8);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int x = tid + 256 * u, r = x / 16, c = x % 16;
        const bool ok = r < len;
        const float f = ok ? a.scale * __expf(gv[u]) : 0.f;
        const uint32_t qw[4] = {qv[u].x, qv[u].y, qv[u].z, qv[u].w};
        uint32_t qo[4];
#pragma unroll
        for (int e = 0; e < 4; e++) qo[e] = pack2<DT>(unpack_lo<DT>(qw[e]) * f, unpack_hi<DT>(qw[e]) * f);
        *(uint4 *)(sm.qg + sw<128>(r, c * 8)) = make_uint4(qo[0], qo[1], qo[2], qo[3]);
        *(uint4 *)(sm.dO + sw<128>(r, c * 8)) = ok ? dv[u] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int x = tid + 256 * u, r = x / 8, c = x % 8;
        *(uint4 *)(sm.aq + sw<64>(r, c * 8)) = av[u];
    }
    __syncthreads();
    // dO as B fragments (k = token, col = state column)
    Frag8 bo[4];
#pragma unroll
    for (int st = 0; st < 4; st++) bo[st] = lds_tr_sw<128>(sm.dO, st * 16, wave * 32, lane);
    // Aqk^T dO (rows = tokens j), then as B fragments of W^T (.), negated
    Frag8 nd[4];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        f32x16_t x = zero16();
#pragma unroll
        for (int st = 0; st < 4; st++)
            x = mfma32<DT>(lds_tr_sw<64>(sm.aq, st * 16, t * 32, lane), bo[st], x);
        nd[2 * t] = c_frag<DT>(x, 0, -1.f);
        nd[2 * t + 1] = c_frag<DT>(x, 1, -1.f);
    }
    // F = (gamma scale Q)^T dO - W^T (Aqk^T dO): rows dk (4 tiles), stored in the product
    // layout in the dtype: [dv tile][dk tile][lane][16]
    uint16_t *fo = w.F + ch * kD * kD + (size_t)wave * 4 * 64 * 16;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        f32x16_t x = zero16();
#pragma unroll
        for (int st = 0; st < 4; st++) {
            x = mfma32<DT>(lds_tr_sw<128>(sm.qg, st * 16, r * 32, lane), bo[st], x);
            x = mfma32<DT>(wa[r][st], nd[st], x);
        }
        uint4 *o = (uint4 *)(fo + ((size_t)r * 64 + lane) * 16);
        o[0] = c_frag<DT>(x, 0).u;
        o[1] = c_frag<DT>(x, 1).u;
    }
}

// The state gradient, backwards over a sequence's chunks, with the rows of dS split over a pair
// of wavefronts per column block (as the forward's state pass): each forms its part of X = (lam K) dS_{c+1} over its 64 rows, the pair
// swaps the parts through LDS, and each updates its own rows.
struct BwdHalfOps {
    Frag8 kr[2][4];  // lam K: token tile t, dk step 4 p + st
    Frag8 wt[2][4];  // W^T: dk tile 2 p + r, token step st
    Frag8 f[2][2];   // F: dk tile 2 p + r, the lane's 16 values as two 8-value halves
    float glast;
};

template <int DT>
__global__ __launch_bounds__(128, 1) void gdr_bwd_state2(GdrArgs a, MfmaWs w, const float *d_final,
                                                        float *dh0) {
    __shared__ __align__(16) float4 xch[2][2][2][4][64];  // [parity][wavefront][token tile][i / 4][lane]
    int64_t sh;
    int blk;
    if (!state_item(blockIdx.x, w.nsh, w.seq_order, a.H, &sh, &blk)) return;
    const int64_t s = sh / a.H, h = sh % a.H;
    const int lane = threadIdx.x & 63;
    const int p = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // row half
    const int col = lane & 31;
    const int c0 = w.seq_chunk0[s], c1 = w.seq_chunk0[s + 1];
    const int dv = blk * 32 + col;
    // dS_p: tile r holds rows 64 p + 32 r + crow(i) of column dv
    f32x16_t D[2];
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            {
                const int row = p * 64 + r * 32 + crow(i, lane);
                D[r][i] = d_final && row < a.Dk && dv < a.Dv
                              ? d_final[sh * a.Dk * a.Dv + row * a.Dv + dv] : 0.f;
            }
    // I's rows 16 u + [0, 16) as the A operand against an output-layout tile's 8-value half u
    // as the B operand (lane l's B slot j is row crow(8 u + j, l) at hardware k = 8 (l / 32) + j):
    // the product adds the tile, exactly in f32
    Frag8 ident[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const uint16_t one = DT == DM_BF16 ? 0x3F80 : 0x3C00;
        uint16_t e[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            e[j] = (lane & 31) == 16 * u + 8 * (j / 4) + 4 * (lane >> 5) + (j % 4) ? one : 0;
        ident[u].u = make_uint4(e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16,
                                e[4] | (uint32_t)e[5] << 16, e[6] | (uint32_t)e[7] << 16);
    }
    // a chunk's operands in two parts: lam K and F with G_last (free once X and F's products
    // are issued) and W^T (free once the update is issued); a chunk before the sequence's first
    // loads the first again (every call the same loads)
    auto load_kf = [&](int c, BwdHalfOps &x) __attribute__((always_inline)) {
        c = c >= c0 ? c : c0;
        const int64_t ch = (int64_t)c * a.H + h;
        const uint16_t *kr = w.Krf + ch * kC * kD;
        const uint16_t *f = w.F + ch * kD * kD + (size_t)blk * 4 * 64 * 16;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int st = 0; st < 4; st++)
                x.kr[t][st].u = *(const uint4 *)(kr + ((t * 8 + p * 4 + st) * 64 + lane) * 8);
#pragma unroll
        for (int r = 0; r < 2; r++) {
            x.f[r][0].u = *(const uint4 *)(f + ((size_t)(p * 2 + r) * 64 + lane) * 16);
            x.f[r][1].u = *(const uint4 *)(f + ((size_t)(p * 2 + r) * 64 + lane) * 16 + 8);
        }
        x.glast = w.G[ch * kC + kC - 1];
    };
    auto load_w = [&](int c, BwdHalfOps &x) __attribute__((always_inline)) {
        c = c >= c0 ? c : c0;
        const int64_t ch = (int64_t)c * a.H + h;
        const uint16_t *wt = w.WTf + ch * kC * kD;
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int st = 0; st < 4; st++)
                x.wt[r][st].u = *(const uint4 *)(wt + (((p * 2 + r) * 4 + st) * 64 + lane) * 8);
    };
    // chunk c's step on the operands in x, which then load chunk cn's
    auto step = [&](int c, BwdHalfOps &x, int cn) __attribute__((always_inline)) {
        const int64_t ch = (int64_t)c * a.H + h;
        // this half of dS after the chunk, kept for the gradients as S is in Sf
        Frag8 df[4];
        uint16_t *dso = w.dSf + ch * kD * kD + (size_t)blk * 8 * 64 * 8;
#pragma unroll
        for (int st = 0; st < 4; st++) {
            df[st] = c_frag<DT>(D[st / 2], st % 2);
            *(uint4 *)(dso + ((p * 4 + st) * 64 + lane) * 8) = df[st].u;
        }
        // this half's part of X = (lam K) dS_{c+1}
        f32x16_t X[2];
#pragma unroll
        for (int t = 0; t < 2; t++) X[t] = zero16();
#pragma unroll
        for (int st = 0; st < 4; st++)
#pragma unroll
            for (int t = 0; t < 2; t++) X[t] = mfma32<DT>(x.kr[t][st], df[st], X[t]);
        // dS_c = exp(G_last) dS_{c+1} + F - W^T X on this half's rows: the decay on the vector
        // unit and F by identity products while X's products run
        const float gl = __expf(x.glast);
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int i = 0; i < 16; i++) D[r][i] *= gl;
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int u = 0; u < 2; u++) D[r] = mfma32<DT>(ident[u], x.f[r][u], D[r]);
        load_kf(cn, x);
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                xch[c & 1][p][t][g][lane] =
                    make_float4(X[t][4 * g], X[t][4 * g + 1], X[t][4 * g + 2], X[t][4 * g + 3]);
        __syncthreads();
        // -X from the two shares: each wavefront reads the other's (x + y = y + x exactly, so
        // both wavefronts form the same values)
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 y = xch[c & 1][p ^ 1][t][g][lane];
                X[t][4 * g] = -X[t][4 * g] - y.x;
                X[t][4 * g + 1] = -X[t][4 * g + 1] - y.y;
                X[t][4 * g + 2] = -X[t][4 * g + 2] - y.z;
                X[t][4 * g + 3] = -X[t][4 * g + 3] - y.w;
            }
        Frag8 nx[4];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            nx[2 * t] = c_frag<DT>(X[t], 0);
            nx[2 * t + 1] = c_frag<DT>(X[t], 1);
        }
#pragma unroll
        for (int st = 0; st < 4; st++)
#pragma unroll
            for (int r = 0; r < 2; r++) D[r] = mfma32<DT>(x.wt[r][st], nx[st], D[r]);
        load_w(cn, x);
    };
    BwdHalfOps oa, ob;
    if (c0 < c1) {
        load_kf(c1 - 1, oa);
        load_w(c1 - 1, oa);
        load_kf(c1 - 2, ob);
        load_w(c1 - 2, ob);
    }
    // two chunks a pass, backwards, each register set loading the chunk two before; an odd
    // first chunk after the loop (every pass through the loop issues the same loads)
    int c = c1 - 1;
    for (; c - 1 >= c0; c -= 2) {
        step(c, oa, c - 2);
        step(c - 1, ob, c - 3);
    }
    if (c >= c0) step(c, oa, c - 2);
    if (dh0) {
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int row = p * 64 + r * 32 + crow(i, lane);
                if (row < a.Dk && dv < a.Dv) dh0[sh * a.Dk * a.Dv + row * a.Dv + dv] = D[r][i];
            }
    }
}

// The gradients of one (chunk, head). Wave w owns columns 32 w + [0, 32) of dq, dk, dv (all 64
// tokens) and the 32x32 tile (w / 2, w % 2) of the 64x64 intermediates. LDS in two phases:
// first S^T, dS^T, V'^T and dO (the products over the state columns), then Q, K, V, T and the
// token-by-token intermediates; dV'^T and Aqk live through both.
namespace bl {
constexpr int ST = 0, DST = 34816, VPT = 69632, DOB = 88064, DVPT = 105472, AQ = 123904;
constexpr int QB = 0, KB = 17408, VB = 34816, DWT = 52224, TB = 70656, M1T = 79872, DTT = 89088;
constexpr int M2T = 133120, M3BT = 142336;      // m2^T, later m3^T; m3b^T
constexpr int DVLO = M2T;                       // dV'^T's rounding residual, until m2^T
constexpr int TOKF = 151552;                    // G, gamma, lam, beta, qi, ki [64] f32
constexpr int RED = TOKF + 6 * 256;             // 8 floats
constexpr int PART = RED + 32;                  // 8 x [4][64] f32 partial sums
constexpr int BYTES = PART + 8 * 1024;
}  // namespace bl
static_assert(bl::DTT + kC * kT * 2 <= bl::DVPT && bl::AQ + kC * kT * 2 <= bl::M2T, "phases");
static_assert(bl::BYTES <= 160 * 1024, "LDS");
static_assert(kC * kR * 2 <= bl::TOKF - bl::M2T && kC * kR * 2 <= bl::DTT + kC * kT * 2 - bl::TB &&
                  kC * kR * 2 <= bl::TB - bl::DWT,
              "output rows in dead regions");

#ifdef DM_TRACE_GRADS
// profiling aid (built only with -DDM_TRACE_GRADS=<chunk x head>): clock stamps of thread 0 of
// that item at the kernel's barriers
__device__ uint64_t dm_trace_grads[32];
#define DM_GSTAMP(k)                                                     \
    do {                                                                \
        if (ch == (DM_TRACE_GRADS) && threadIdx.x == 0)                 \
            dm_trace_grads[k] = __builtin_readcyclecounter();           \
    } while (0)
extern "C" int dm_debug_trace_grads(void *host, size_t bytes) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(dm_trace_grads), bytes) == hipSuccess ? 0 : 1;
}
#else
#define DM_GSTAMP(k) \
    do {             \
    } while (0)
#endif

// A 16-bit tile's values at a product output's positions (rows r0 + crow(i, lane), column
// c0 + lane % 32), as f32: two transposed reads (ds_read_b64_tr_b16 hands lane l the rows
// r0 + 8 j + 4 (l / 32) + e of its column in slot 4 j + e, i.e. rows crow(i) for i < 8) in place
// of 16 two-byte reads.
template <int DT>
__device__ __forceinline__ void tile_at_out(const uint16_t *t, int stride, int r0, int c0, int lane,
                                            float (&v)[16]) {
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const Frag8 f = lds_tr_frag(t, stride, r0 + 16 * hh, c0, lane);
        const uint32_t w4[4] = {f.u.x, f.u.y, f.u.z, f.u.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[8 * hh + 2 * e] = unpack_lo<DT>(w4[e]);
            v[8 * hh + 2 * e + 1] = unpack_hi<DT>(w4[e]);
        }
    }
}

template <int DT>
__global__ __launch_bounds__(512, 1) void gdr_bwd_grads(GdrArgs a, MfmaWs w, const void *d_out,
                                                        void *dq, void *dk, void *dv, void *dg,
                                                        void *dbeta) {
    __shared__ __align__(16) char smem[bl::BYTES];
    const int64_t ch = blockIdx.x, n = ch / a.H, h = ch % a.H;
    const int len = w.chunk_len[n];
    if (len == 0) return;
    const int64_t tok0 = w.chunk_tok0[n];
    const int tid = threadIdx.x, lane = tid & 63;
    DM_GSTAMP(0);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, half = lane >> 5;
    // wavefront w: columns 32 (w % 4) + [0, 32) of dq, dk, dv at tokens 32 (w / 4) + [0, 32);
    // and the 32x32 tile ((w / 2) % 2, w % 2) of the 64x64 intermediates: dT on wavefronts 4-7,
    // the others on wavefronts 0-3
    const int cw = wave & 3, tw = wave >> 2;
    const bool tilew = wave < 4;
    const int ti = (wave >> 1) & 1, tj = wave & 1;
    auto U16 = [&](int off) { return (uint16_t *)(smem + off); };
    auto F32 = [&](int off) { return (float *)(smem + off); };
    uint16_t *sST = U16(bl::ST), *sDST = U16(bl::DST), *sVPT = U16(bl::VPT), *sDOB = U16(bl::DOB);
    uint16_t *sDVPT = U16(bl::DVPT), *sAQ = U16(bl::AQ), *sDVLO = U16(bl::DVLO);
    float *tG = F32(bl::TOKF), *tGam = tG + 64, *tLam = tG + 128, *tBet = tG + 192,
          *tQi = tG + 256, *tKi = tG + 320;
    float *pGam = F32(bl::PART), *pU = pGam + 256, *pS = pGam + 512, *pBet = pGam + 768,
          *pGr = pGam + 1024, *pGc = pGam + 1280, *pSq = pGam + 1536, *pSk = pGam + 1792;

    // dV''s first products' operands, (lam K) and dS_{c+1} fragments, loaded with phase 1's rows
    // (they are used straight from registers after its barrier)
    Frag8 dv_ka[8], dv_db[8];
    {
        const uint16_t *kr = w.Krf + ch * kC * kD;
        const uint16_t *dsf = w.dSf + ch * kD * kD + (size_t)cw * 8 * 64 * 8;
#pragma unroll
        for (int st = 0; st < 8; st++) {
            dv_ka[st].u = *(const uint4 *)(kr + ((tw * 8 + st) * 64 + lane) * 8);
            dv_db[st].u = *(const uint4 *)(dsf + (st * 64 + lane) * 8);
        }
    }
    // ---- phase 1: per-token values; S^T, dS^T, V'^T from their fragments; dO, Aqk rows ----
    {
        const uint16_t *sf = w.Sf + ch * kD * kD, *dsf = w.dSf + ch * kD * kD;
        const uint16_t *vf = w.Vf + ch * kC * kD, *dob = (const uint16_t *)d_out;
        // every load issued before the first store
        uint4 s1[4], s2[4], s3[2], s4[2], s5;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s1[i] = *(const uint4 *)(sf + (size_t)(tid + 512 * i) * 8);
            s2[i] = *(const uint4 *)(dsf + (size_t)(tid + 512 * i) * 8);
        }
#pragma unroll
        for (int i = 0; i < 2; i++) s3[i] = *(const uint4 *)(vf + (size_t)(tid + 512 * i) * 8);
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int x = tid + 512 * u, r = x / 16, c = x % 16;
            s4[u] = c * 8 < a.Dv
                        ? *(const uint4 *)(dob + o_at(a, tok0 + (r < len ? r : len - 1), h) + c * 8)
                        : zero4();
        }
        s5 = *(const uint4 *)(w.Aqk + ch * kC * kC + (tid / 8) * kC + (tid % 8) * 8);
        // per-token values (after the rows' loads: these reads wait on the memory counter)
        if (tid < kC) {
            const float gv = w.G[ch * kC + tid];
            tG[tid] = gv;
            tGam[tid] = __expf(gv);
            tLam[tid] = __expf(w.G[ch * kC + kC - 1] - gv);
            tBet[tid] = tid < len ? ld_any(a.beta_dt, a.beta, b_at(a, tok0 + tid, h)) : 0.f;
        }
        // fragment (dv tile p, dk step st), lane l: column dv = 32 p + l % 32 (a row of X^T),
        // dk runs 16 st + 4 (l / 32) + [0, 4) and 16 st + 8 + 4 (l / 32) + [0, 4)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int x = tid + 512 * i, f = x / 64, l = x % 64, p = f / 8, st = f % 8;
            const int r = p * 32 + (l & 31), c = st * 16 + (l >> 5) * 4;
            *(uint2 *)(sST + sw<128>(r, c)) = make_uint2(s1[i].x, s1[i].y);
            *(uint2 *)(sST + sw<128>(r, c + 8)) = make_uint2(s1[i].z, s1[i].w);
            *(uint2 *)(sDST + sw<128>(r, c)) = make_uint2(s2[i].x, s2[i].y);
            *(uint2 *)(sDST + sw<128>(r, c + 8)) = make_uint2(s2[i].z, s2[i].w);
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int x = tid + 512 * i, f = x / 64, l = x % 64, p = f / 4, st = f % 4;
            const int r = p * 32 + (l & 31), c = st * 16 + (l >> 5) * 4;
            *(uint2 *)(sVPT + sw<64>(r, c)) = make_uint2(s3[i].x, s3[i].y);
            *(uint2 *)(sVPT + sw<64>(r, c + 8)) = make_uint2(s3[i].z, s3[i].w);
        }
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int x = tid + 512 * u, r = x / 16, c = x % 16;
            *(uint4 *)(sDOB + sw<128>(r, c * 8)) = r < len ? s4[u] : make_uint4(0, 0, 0, 0);
        }
        *(uint4 *)(sAQ + sw<64>(tid / 8, (tid % 8) * 8)) = s5;
        for (int x = tid; x < 8 * 256; x += 512) pGam[x] = 0.f;
    }
    __syncthreads();
    DM_GSTAMP(1);
    // dV' = (lam K) dS_{c+1} + Aqk^T dO for the wave's 32 columns and 32 tokens, stored as dV'^T
    {
        const int t = tw;
        {
            f32x16_t x = zero16();
#pragma unroll
            for (int st = 0; st < 8; st++) x = mfma32<DT>(dv_ka[st], dv_db[st], x);
#pragma unroll
            for (int st = 0; st < 4; st++)
                x = mfma32<DT>(lds_tr_sw<64>(sAQ, st * 16, t * 32, lane),
                               lds_tr_sw<128>(sDOB, st * 16, cw * 32, lane), x);
            store_ct_sw<DT, 64>(sDVPT, t * 32, cw * 32, x, lane);
            // and what the rounding left, for T^T dV' (d beta's largest term)
#pragma unroll
            for (int i = 0; i < 16; i++) x[i] -= round_to<DT>(x[i]);
            store_ct_sw<DT, 64>(sDVLO, t * 32, cw * 32, x, lane);
        }
    }
    __syncthreads();
    DM_GSTAMP(2);
    // (a) d(gamma q) = dO S^T, (e) dkt = V' dS_{c+1}^T, (f) dw = -dV' S^T: the wave's token tile
    // of its 32 dk columns; (b) d attn = dO V'^T on the wave's tile, zero above the diagonal
    f32x16_t dqg, dkt, dw, datt = zero16();
    {
        const int t = tw;
        dqg = dkt = dw = zero16();
#pragma unroll
        for (int st = 0; st < 8; st++) {
            const Frag8 bs = lds_tr_sw<128>(sST, st * 16, cw * 32, lane);
            dqg = mfma32<DT>(row_frag_sw<128>(sDOB, t * 32, st * 16, lane), bs, dqg);
            dw = mfma32<DT>(lds_tr_sw<64>(sDVPT, st * 16, t * 32, lane), bs, dw);
            dkt = mfma32<DT>(lds_tr_sw<64>(sVPT, st * 16, t * 32, lane),
                             lds_tr_sw<128>(sDST, st * 16, cw * 32, lane), dkt);
        }
    }
    if (tilew && !(ti == 0 && tj == 1)) {
#pragma unroll
        for (int st = 0; st < 8; st++)
            datt = mfma32<DT>(row_frag_sw<128>(sDOB, ti * 32, st * 16, lane),
                              lds_tr_sw<64>(sVPT, st * 16, tj * 32, lane), datt);
    }
    // <S, dS_{c+1}> over the chunk
    {
        float acc = 0.f;
        for (int x = tid; x < kD * 16; x += 512) {
            const int r = x / 16, c = (x % 16) * 8;
            const uint4 s1 = *(const uint4 *)(sST + sw<128>(r, c)), s2 = *(const uint4 *)(sDST + sw<128>(r, c));
            const uint32_t a1[4] = {s1.x, s1.y, s1.z, s1.w}, a2[4] = {s2.x, s2.y, s2.z, s2.w};
#pragma unroll
            for (int e = 0; e < 4; e++)
                acc += unpack_lo<DT>(a1[e]) * unpack_lo<DT>(a2[e]) + unpack_hi<DT>(a1[e]) * unpack_hi<DT>(a2[e]);
        }
        acc = sum32(acc);
        acc += __shfl_xor(acc, 32, 64);
        if (lane == 0) F32(bl::RED)[wave] = acc;
    }
    __syncthreads();  // phase 1 done: S^T, dS^T, V'^T and dO are dead
    DM_GSTAMP(3);

    // ---- phase 2: Q, K (normalised as the forward did, with the inverse norms), V, T ----
    uint4 q2[2], k2[2], v2[2], t2;
    {
        const uint16_t *qin = (const uint16_t *)a.q, *kin = (const uint16_t *)a.k,
                       *vin = (const uint16_t *)a.v;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int x = tid + 512 * u, r = x / 16, c = x % 16;
            const int64_t tok = tok0 + (r < len ? r : len - 1);
            q2[u] = c * 8 < a.Dk ? *(const uint4 *)(qin + q_at(a, tok, h) + c * 8) : zero4();
            k2[u] = c * 8 < a.Dk ? *(const uint4 *)(kin + k_at(a, tok, h) + c * 8) : zero4();
            v2[u] = c * 8 < a.Dv ? *(const uint4 *)(vin + v_at(a, tok, h) + c * 8) : zero4();
        }
        t2 = *(const uint4 *)(w.Tm + ch * kC * kC + (tid / 8) * kC + (tid % 8) * 8);
    }
    {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int x = tid + 512 * u, r = x / 16, c = x % 16;
            const bool ok = r < len;
            uint4 qv = q2[u], kv = k2[u];
            const uint4 vv = v2[u];
            float qi = 1.f, ki = 1.f;
            if (a.l2norm) {
                const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w}, kw[4] = {kv.x, kv.y, kv.z, kv.w};
                float sq = 0.f, sk = 0.f;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float q0 = unpack_lo<DT>(qw[e]), q1 = unpack_hi<DT>(qw[e]);
                    const float k0 = unpack_lo<DT>(kw[e]), k1 = unpack_hi<DT>(kw[e]);
                    sq += q0 * q0 + q1 * q1;
                    sk += k0 * k0 + k1 * k1;
                }
#pragma unroll
                for (int o = 8; o >= 1; o >>= 1) {
                    sq += __shfl_xor(sq, o, 64);
                    sk += __shfl_xor(sk, o, 64);
                }
                qi = 1.f / sqrtf(sq + 1e-6f);
                ki = 1.f / sqrtf(sk + 1e-6f);
                uint32_t qo[4], ko[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    qo[e] = pack2<DT>(unpack_lo<DT>(qw[e]) * qi, unpack_hi<DT>(qw[e]) * qi);
                    ko[e] = pack2<DT>(unpack_lo<DT>(kw[e]) * ki, unpack_hi<DT>(kw[e]) * ki);
                }
                qv = make_uint4(qo[0], qo[1], qo[2], qo[3]);
                kv = make_uint4(ko[0], ko[1], ko[2], ko[3]);
            }
            // rows past the chunk's tokens are zero (component-wise selects: a select of whole
            // vectors goes through private memory)
            const uint32_t keep = ok ? 0xffffffffu : 0u;
            *(uint4 *)(U16(bl::QB) + sw<128>(r, c * 8)) =
                make_uint4(qv.x & keep, qv.y & keep, qv.z & keep, qv.w & keep);
            *(uint4 *)(U16(bl::KB) + sw<128>(r, c * 8)) =
                make_uint4(kv.x & keep, kv.y & keep, kv.z & keep, kv.w & keep);
            *(uint4 *)(U16(bl::VB) + sw<128>(r, c * 8)) =
                make_uint4(vv.x & keep, vv.y & keep, vv.z & keep, vv.w & keep);
            if (c == 0) {
                tQi[r] = qi;
                tKi[r] = ki;
            }
        }
        *(uint4 *)(U16(bl::TB) + sw<64>(tid / 8, (tid % 8) * 8)) = t2;
    }
    uint16_t *sQB = U16(bl::QB), *sKB = U16(bl::KB), *sVB = U16(bl::VB), *sDWT = U16(bl::DWT);
    uint16_t *sTB = U16(bl::TB), *sM1T = U16(bl::M1T), *sDTT = U16(bl::DTT);
    uint16_t *sM2T = U16(bl::M2T), *sM3BT = U16(bl::M3BT);
    // dw^T (negated: dw = -dV' S^T) and m1^T = (d attn o decay)^T
    store_ct_sw<DT, 64>(sDWT, tw * 32, cw * 32, dw, lane, -1.f);
    if (tilew) {
        f32x16_t m = zero16();
        if (!(ti == 0 && tj == 1)) {
            const int j = tj * 32 + col;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int r = ti * 32 + crow(i, lane);
                if (j > r) datt[i] = 0.f;
                m[i] = datt[i] * (r >= j ? __expf(tG[r] - tG[j]) : 0.f);
            }
        }
        store_ct_sw<DT, 64>(sM1T, ti * 32, tj * 32, m, lane);
    }
    __syncthreads();  // Q, K, V, T, dw^T, m1^T in place
    DM_GSTAMP(4);
    const float scale = a.scale;
    // (d) d attn o attn: + row sums, - column sums into dG
    if (tilew && !(ti == 0 && tj == 1)) {
        const int j = tj * 32 + col;
        float cs = 0.f, p[16], avs[16];
        tile_at_out_sw<DT, 64>(sAQ, ti * 32, tj * 32, lane, avs);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float av = avs[i];
            p[i] = datt[i] * av;
            cs += p[i];
        }
        int rr;
        const float rs = tile_rowsum(p, lane, &rr);
        if (!(lane & 1)) pGr[wave * 64 + ti * 32 + rr] += rs;
        cs += __shfl_xor(cs, 32, 64);
        if (half == 0) pGc[wave * 64 + j] += cs;
    }
    // dq = gamma d(gamma q) + m1 K; dk = lam dkt + scale m1^T Q; d gamma, s partial sums
    f32x16_t dqa, dka, dva;
    {
        const int t = tw;
        float gsum[16], ssum[16], qvs[16], kvs[16];
        tile_at_out_sw<DT, 128>(sQB, t * 32, cw * 32, lane, qvs);
        tile_at_out_sw<DT, 128>(sKB, t * 32, cw * 32, lane, kvs);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = t * 32 + crow(i, lane);
            const float qv = qvs[i], kv = kvs[i];
            gsum[i] = dqg[i] * qv * scale;
            ssum[i] = dkt[i] * kv;
            dqa[i] = tGam[r] * dqg[i];
            dka[i] = tLam[r] * dkt[i];
        }
        {
            int rr;
            const float g1 = tile_rowsum(gsum, lane, &rr), s1 = tile_rowsum(ssum, lane, &rr);
            if (!(lane & 1)) {
                pGam[cw * 64 + t * 32 + rr] += g1;
                pS[cw * 64 + t * 32 + rr] += s1;
            }
        }
        f32x16_t x = zero16();
#pragma unroll
        for (int st = 0; st < 4; st++) {
            dqa = mfma32<DT>(lds_tr_sw<64>(sM1T, st * 16, t * 32, lane),
                             lds_tr_sw<128>(sKB, st * 16, cw * 32, lane), dqa);
            x = mfma32<DT>(row_frag_sw<64>(sM1T, t * 32, st * 16, lane),
                           lds_tr_sw<128>(sQB, st * 16, cw * 32, lane), x);
        }
#pragma unroll
        for (int i = 0; i < 16; i++) dka[i] += scale * x[i];
    }
    // (g) dT = dV' (beta V)^T + dw (beta gamma K)^T on tile (ti, tj), stored as dT^T: wavefronts
    // 4-7 (0-3 have the d attn sums above)
    if (!tilew) {
        f32x16_t c1 = zero16(), c2 = zero16();
#pragma unroll
        for (int st = 0; st < 8; st++) {
            c1 = mfma32<DT>(lds_tr_sw<64>(sDVPT, st * 16, ti * 32, lane),
                            row_frag_sw<128>(sVB, tj * 32, st * 16, lane), c1);
            c2 = mfma32<DT>(lds_tr_sw<64>(sDWT, st * 16, ti * 32, lane),
                            row_frag_sw<128>(sKB, tj * 32, st * 16, lane), c2);
        }
        const int j = tj * 32 + col;
        const float bj = tBet[j], bgj = tBet[j] * tGam[j];
#pragma unroll
        for (int i = 0; i < 16; i++) c1[i] = c1[i] * bj + c2[i] * bgj;
        store_ct_sw<DT, 64>(sDTT, ti * 32, tj * 32, c1, lane);
    }
    // (h) dvb = T^T dV', dkbg = T^T dw: dv = beta dvb; dk += beta gamma dkbg; sums for d beta,
    // d gamma
    {
        const int t = tw;
        f32x16_t xb = zero16(), xk = zero16();
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const Frag8 ta = lds_tr_sw<64>(sTB, st * 16, t * 32, lane);
            xb = mfma32<DT>(ta, row_frag_sw<64>(sDVPT, cw * 32, st * 16, lane), xb);
            xb = mfma32<DT>(ta, row_frag_sw<64>(sDVLO, cw * 32, st * 16, lane), xb);
            xk = mfma32<DT>(ta, row_frag_sw<64>(sDWT, cw * 32, st * 16, lane), xk);
        }
        float bs[16], us[16], vvs[16], kvs[16];
        tile_at_out_sw<DT, 128>(sVB, t * 32, cw * 32, lane, vvs);
        tile_at_out_sw<DT, 128>(sKB, t * 32, cw * 32, lane, kvs);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = t * 32 + crow(i, lane);
            const float vv = vvs[i], kv = kvs[i];
            dva[i] = tBet[r] * xb[i];
            dka[i] += tBet[r] * tGam[r] * xk[i];
            bs[i] = xb[i] * vv;
            us[i] = xk[i] * kv;
        }
        {
            int rr;
            const float b1 = tile_rowsum(bs, lane, &rr), u1 = tile_rowsum(us, lane, &rr);
            if (!(lane & 1)) {
                pBet[cw * 64 + t * 32 + rr] += b1;
                pU[cw * 64 + t * 32 + rr] += u1;
            }
        }
    }
    __syncthreads();  // dT^T complete
    DM_GSTAMP(5);
    // (i) m2 = T^T dT on the wave's tile (a, b) = (ti, tj), stored as m2^T
    if (tilew) {
        f32x16_t m2 = zero16();
#pragma unroll
        for (int st = 0; st < 4; st++)
            m2 = mfma32<DT>(lds_tr_sw<64>(sTB, st * 16, ti * 32, lane),
                            row_frag_sw<64>(sDTT, tj * 32, st * 16, lane), m2);
        store_ct_sw<DT, 64>(sM2T, ti * 32, tj * 32, m2, lane);
    }
    __syncthreads();
    DM_GSTAMP(6);
    // dA = -(m2 T^T) strictly below the diagonal on tile (a, c) = (ti, tj); the recomputed
    // A = beta (K K^T) o decay for the gate's sums; m3 = dA o decay
    f32x16_t m3 = zero16(), m3b = zero16();
    if (tilew && !(ti == 0 && tj == 1)) {
        f32x16_t da = zero16(), kk = zero16();
#pragma unroll
        for (int st = 0; st < 4; st++)
            da = mfma32<DT>(lds_tr_sw<64>(sM2T, st * 16, ti * 32, lane),
                            row_frag_sw<64>(sTB, tj * 32, st * 16, lane), da);
#pragma unroll
        for (int st = 0; st < 8; st++)
            kk = mfma32<DT>(row_frag_sw<128>(sKB, ti * 32, st * 16, lane),
                            row_frag_sw<128>(sKB, tj * 32, st * 16, lane), kk);
        const int j = tj * 32 + col;
        float cs = 0.f, p[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = ti * 32 + crow(i, lane);
            const bool lower = r > j;
            const float d = lower ? -da[i] : 0.f;
            const float dec = lower ? __expf(tG[r] - tG[j]) : 0.f;
            const float am = tBet[r] * kk[i] * dec;
            p[i] = d * am;
            cs += p[i];
            m3[i] = d * dec;
            m3b[i] = m3[i] * tBet[r];
        }
        {
            int rr;
            const float rs = tile_rowsum(p, lane, &rr);
            if (!(lane & 1)) pGr[wave * 64 + ti * 32 + rr] += rs;
        }
        cs += __shfl_xor(cs, 32, 64);
        if (half == 0) pGc[wave * 64 + j] += cs;
    }
    __syncthreads();  // m2^T dead: m3^T takes its place
    DM_GSTAMP(7);
    if (tilew) {
        store_ct_sw<DT, 64>(sM2T, ti * 32, tj * 32, m3, lane);
        store_ct_sw<DT, 64>(sM3BT, ti * 32, tj * 32, m3b, lane);
    }
    __syncthreads();
    DM_GSTAMP(8);
    // (j) dkbeta = m3 K: dk += beta dkbeta; d beta sums; dk += m3^T (beta K)
    {
        const int t = tw;
        f32x16_t xb = zero16(), xt = zero16();
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const Frag8 kb = lds_tr_sw<128>(sKB, st * 16, cw * 32, lane);
            xb = mfma32<DT>(lds_tr_sw<64>(sM2T, st * 16, t * 32, lane), kb, xb);
            xt = mfma32<DT>(row_frag_sw<64>(sM3BT, t * 32, st * 16, lane), kb, xt);
        }
        float bs[16], kvs[16];
        tile_at_out_sw<DT, 128>(sKB, t * 32, cw * 32, lane, kvs);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = t * 32 + crow(i, lane);
            const float kv = kvs[i];
            dka[i] += tBet[r] * xb[i] + xt[i];
            bs[i] = xb[i] * kv;
        }
        {
            int rr;
            const float b1 = tile_rowsum(bs, lane, &rr);
            if (!(lane & 1)) pBet[cw * 64 + t * 32 + rr] += b1;
        }
    }
    // (m) the l2 normalisation's sums: <qn, scale dq>, <kn, dk> per token
    if (a.l2norm) {
        {
            const int t = tw;
            float qs[16], ks[16], qvs[16], kvs[16];
            tile_at_out_sw<DT, 128>(sQB, t * 32, cw * 32, lane, qvs);
            tile_at_out_sw<DT, 128>(sKB, t * 32, cw * 32, lane, kvs);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float qv = qvs[i], kv = kvs[i];
                qs[i] = qv * dqa[i] * scale;
                ks[i] = kv * dka[i];
            }
            {
                int rr;
                const float q1 = tile_rowsum(qs, lane, &rr), k1 = tile_rowsum(ks, lane, &rr);
                if (!(lane & 1)) {
                    pSq[cw * 64 + t * 32 + rr] = q1;
                    pSk[cw * 64 + t * 32 + rr] = k1;
                }
            }
        }
    }
    __syncthreads();
    DM_GSTAMP(9);
    // per token: dG, then dg = its reverse cumulative sum; d beta
    if (wave == 0) {
        const int i = lane;
        float gam = 0.f, u = 0.f, s = 0.f, bet = 0.f, gr = 0.f;
#pragma unroll
        for (int x = 0; x < 4; x++) {
            gam += pGam[x * 64 + i];
            u += pU[x * 64 + i];
            s += pS[x * 64 + i];
            bet += pBet[x * 64 + i];
            gr += pGr[x * 64 + i] - pGc[x * 64 + i];
        }
        gam += tBet[i] * u;
        bet += tGam[i] * u;
        const float ls = tLam[i] * s;
        float dG = gr - ls + gam * tGam[i];
        float lam_sum = ls;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) lam_sum += __shfl_xor(lam_sum, o, 64);
        const float* red = F32(bl::RED);
        const float sds = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
        if (i == kC - 1) dG += lam_sum + sds * __expf(tG[kC - 1]);
        // reverse inclusive scan
        float x = dG;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_down(x, o, 64);
            if (i + o < 64) x += y;
        }
        if (i < len) {
            const int64_t tk = (tok0 + i) * a.H + h;
            st_any(a.g_dt, dg, tk, x);
            st_any(a.beta_dt, dbeta, tk, bet);
        }
        if (a.l2norm) {
            float sq = 0.f, sk = 0.f;
#pragma unroll
            for (int x2 = 0; x2 < 4; x2++) {
                sq += pSq[x2 * 64 + i];
                sk += pSk[x2 * 64 + i];
            }
            pSq[i] = sq;
            pSk[i] = sk;
        }
    }
    __syncthreads();
    DM_GSTAMP(10);
    // dq, dk (the scale and the l2 normalisation undone), dv: staged as rows in LDS (regions
    // dead by now), then stored 16 bytes per lane
    uint16_t *oq = U16(bl::DWT), *ok_ = U16(bl::M2T), *ov = U16(bl::TB);
    {
        const int t = tw;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = t * 32 + crow(i, lane);
            const int c = cw * 32 + col;
            float qo = dqa[i] * scale, ko = dka[i];
            if (a.l2norm) {
                const uint16_t qb = sQB[sw<128>(r, c)], kb = sKB[sw<128>(r, c)];
                const float qv = (DT == DM_BF16) ? __uint_as_float((uint32_t)qb << 16)
                                                 : (float)__builtin_bit_cast(_Float16, qb);
                const float kv = (DT == DM_BF16) ? __uint_as_float((uint32_t)kb << 16)
                                                 : (float)__builtin_bit_cast(_Float16, kb);
                qo = tQi[r] * (qo - qv * pSq[r]);
                ko = tKi[r] * (ko - kv * pSk[r]);
            }
            oq[r * kR + c] = (uint16_t)(pack2<DT>(qo, 0.f) & 0xffffu);
            ok_[r * kR + c] = (uint16_t)(pack2<DT>(ko, 0.f) & 0xffffu);
            ov[r * kR + c] = (uint16_t)(pack2<DT>(dva[i], 0.f) & 0xffffu);
        }
    }
    __syncthreads();
    DM_GSTAMP(11);
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int x = tid + 512 * u, r = x / 16, c = x % 16;
        if (r < len) {
            const int64_t ok = ((tok0 + r) * a.H + h) * a.Dk + c * 8;
            const int64_t ov_ = ((tok0 + r) * a.H + h) * a.Dv + c * 8;
            if (c * 8 < a.Dk) {
                *(uint4 *)((uint16_t *)dq + ok) = *(const uint4 *)(oq + r * kR + c * 8);
                *(uint4 *)((uint16_t *)dk + ok) = *(const uint4 *)(ok_ + r * kR + c * 8);
            }
            if (c * 8 < a.Dv) *(uint4 *)((uint16_t *)dv + ov_) = *(const uint4 *)(ov + r * kR + c * 8);
        }
    }
    DM_GSTAMP(12);
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------

bool gdr_mfma_takes(const dm_gdr_desc *d) {
    // (16-byte row loads and stores; the base pointers' alignment is checked by the entry
    // points, which refuse misaligned ones) head widths below 128 run the same products with the columns past the width held at
    // zero (loaded as zeros, never stored): a zero key or query column adds nothing to any
    // product or norm, and the state's rows and columns past the widths stay zero
    return (d->dtype == DM_BF16 || d->dtype == DM_F16) && d->dk % 8 == 0 && d->dv % 8 == 0 &&
           d->dk >= 8 && d->dv >= 8 && d->dk <= kD && d->dv <= kD && gdr_strides_16b(d);
}

size_t gdr_mfma_fwd_workspace(const dm_gdr_desc *d) { return mfma_layout(d, nullptr, nullptr); }

#ifdef DM_TRACE_STATE
extern "C" int dm_debug_trace_state(void *host, size_t bytes) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(dm_trace_state), bytes) == hipSuccess ? 0 : 1;
}
extern "C" int dm_debug_trace_out(void *host, size_t bytes) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(dm_trace_out), bytes) == hipSuccess ? 0 : 1;
}
#endif

// LDS the state passes' launches take in all (their own plus a dynamic reservation), so that one
// workgroup takes a compute unit: a chain step whose wavefronts share the compute unit's load,
// LDS and issue with another workgroup's took 4,000-6,500 cycles against 2,600 alone, and the
// longest chains, taken first, decide the pass's time (config 4: 265 -> 227 us).
constexpr unsigned kStateLds = 82 * 1024;
// the dynamic LDS a launch of `kernel` adds to its own to take kStateLds (worked out, and the
// kernel's dynamic-LDS limit raised, once per device and kernel)
static unsigned state_lds_of(const void *kernel) {
    static std::mutex mu;
    static std::vector<std::tuple<int, const void *, unsigned>> known;
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lock(mu);
    for (const auto &e : known)
        if (std::get<0>(e) == dev && std::get<1>(e) == kernel) return std::get<2>(e);
    hipFuncAttributes fa{};
    if (hipFuncGetAttributes(&fa, kernel) != hipSuccess) return 0;
    const unsigned own = (unsigned)fa.sharedSizeBytes;
    unsigned extra = own >= kStateLds ? 0u : kStateLds - own;
    if (extra > 64 * 1024 &&
        hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)extra) !=
            hipSuccess)
        extra = 0;  // (then workgroups may share a compute unit: slower, still correct)
    known.emplace_back(dev, kernel, extra);
    return extra;
}
template <typename K>
static unsigned state_lds(K kernel) {
    return state_lds_of(reinterpret_cast<const void *>(kernel));
}

int launch_gdr_mfma_fwd(const dm_gdr_desc *d, const void *q, const void *k, const void *v,
                        const void *g, const void *beta, const float *h0, void *out,
                        float *final_state, void *workspace, hipStream_t st) {
    MfmaWs w;
    mfma_layout(d, (char *)workspace, &w);
    const GdrArgs a = gdr_args(d, q, k, v, g, beta);
    const int64_t nc = gdr_chunk_bound(d), S = gdr_nseq(d);
    int rc = launch_plan(d, w.seq_chunk0, w.chunk_seq, w.chunk_tok0, w.chunk_len, st, w.seq_order);
    if (rc) return rc;
    const unsigned chunks = (unsigned)(nc * d->h), seqs = (unsigned)(S * d->h);
    if (d->dtype == DM_BF16) {
        {
            KernelTimer t(DM_KERNEL_GDR_PREP, st);
            if (chunks) gdr_mfma_prep<DM_BF16><<<chunks, 256, 0, st>>>(a, w);
        }
        {
            KernelTimer t(DM_KERNEL_GDR_STATE, st);
            gdr_mfma_state2<DM_BF16, kStateParts, true><<<(unsigned)state_grid(seqs), 64 * kStateParts + 128, state_lds(gdr_mfma_state2<DM_BF16, kStateParts, true>), st>>>(a, w, h0, final_state, out);
        }
    } else {
        {
            KernelTimer t(DM_KERNEL_GDR_PREP, st);
            if (chunks) gdr_mfma_prep<DM_F16><<<chunks, 256, 0, st>>>(a, w);
        }
        {
            KernelTimer t(DM_KERNEL_GDR_STATE, st);
            gdr_mfma_state2<DM_F16, kStateParts, true><<<(unsigned)state_grid(seqs), 64 * kStateParts + 128, state_lds(gdr_mfma_state2<DM_F16, kStateParts, true>), st>>>(a, w, h0, final_state, out);
        }
    }
    probe_add(DM_PROBE_GDR_CHUNK_FWD, 4);
    probe_add(DM_PROBE_GDR_CHUNK_FWD_MFMA, 4);
    DM_LAUNCH_CHECK("chunk_gated_delta_rule: MFMA launch");
    return DM_OK;
}

size_t gdr_mfma_bwd_workspace(const dm_gdr_desc *d) {
    return mfma_layout(d, nullptr, nullptr, true);
}

// plan -> prep (with T, lam K and W^T for the backward) -> the forward's state pass (S and V'
// per chunk) -> F per chunk -> the state gradient's pass (dS per chunk, dh0) -> the gradients
template <int DT>
static void gdr_mfma_bwd_kernels(const GdrArgs &a, const MfmaWs &w, unsigned chunks,
                                 unsigned seqs, const float *h0, const void *d_out,
                                 const float *d_final, void *dq, void *dk, void *dv, void *dg,
                                 void *dbeta, float *dh0, hipStream_t st) {
    {
        KernelTimer t(DM_KERNEL_GDR_PREP, st);
        if (chunks) gdr_mfma_prep<DT><<<chunks, 256, 0, st>>>(a, w);
    }
    {
        KernelTimer t(DM_KERNEL_GDR_STATE, st);
        gdr_mfma_state2<DT, kStateParts, false><<<(unsigned)state_grid(seqs), 64 * kStateParts, state_lds(gdr_mfma_state2<DT, kStateParts, false>), st>>>(a, w, h0, nullptr, nullptr);
    }
    {
        KernelTimer t(DM_KERNEL_GDR_BWD_PRE, st);
        if (chunks) gdr_bwd_pre<DT><<<chunks, 256, 0, st>>>(a, w, d_out);
    }
    {
        KernelTimer t(DM_KERNEL_GDR_BWD_STATE, st);
        gdr_bwd_state2<DT><<<(unsigned)state_grid(seqs), 128, state_lds(gdr_bwd_state2<DT>), st>>>(a, w, d_final, dh0);
    }
    {
        KernelTimer t(DM_KERNEL_GDR_BWD_GRADS, st);
        if (chunks)
            gdr_bwd_grads<DT><<<chunks, 512, 0, st>>>(a, w, d_out, dq, dk, dv, dg, dbeta);
    }
}

int launch_gdr_mfma_bwd(const dm_gdr_desc *d, const void *q, const void *k, const void *v,
                        const void *g, const void *beta, const float *h0, const void *d_out,
                        const float *d_final, void *dq, void *dk, void *dv, void *dg,
                        void *dbeta, float *dh0, void *workspace, hipStream_t st) {
    MfmaWs w;
    mfma_layout(d, (char *)workspace, &w, true);
    const GdrArgs a = gdr_args(d, q, k, v, g, beta);
    const int64_t nc = gdr_chunk_bound(d), S = gdr_nseq(d);
    int rc = launch_plan(d, w.seq_chunk0, w.chunk_seq, w.chunk_tok0, w.chunk_len, st, w.seq_order);
    if (rc) return rc;
    const unsigned chunks = (unsigned)(nc * d->h), seqs = (unsigned)(S * d->h);
    if (d->dtype == DM_BF16)
        gdr_mfma_bwd_kernels<DM_BF16>(a, w, chunks, seqs, h0, d_out, d_final, dq, dk, dv, dg,
                                      dbeta, dh0, st);
    else
        gdr_mfma_bwd_kernels<DM_F16>(a, w, chunks, seqs, h0, d_out, d_final, dq, dk, dv, dg,
                                     dbeta, dh0, st);
    probe_add(DM_PROBE_GDR_CHUNK_BWD, 6);
    probe_add(DM_PROBE_GDR_CHUNK_BWD_MFMA, 6);
    DM_LAUNCH_CHECK("chunk_gated_delta_rule_backward: MFMA launch");
    return DM_OK;
}

}  // namespace dm
