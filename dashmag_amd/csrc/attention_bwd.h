// Definitions shared by the MFMA attention backward's translation units (attention_mfma_bwd.hip:
// the passes, the work order, dQ and the dK/dV kernel at head widths 64 and 128;
// attention_bwd_w4.hip: the dK/dV kernel at head width 256, built with its own scheduling
// strategy).
#pragma once

#include "attention_kernels.h"

namespace dm {

constexpr int kRowTile = 32;   // rows per tile of the prep's tile ranges (= the dK/dV step)
constexpr int kKvBlock = 128;  // keys per dK/dV workgroup (32 per wavefront pair)
constexpr int kDqM = 128;      // queries per dQ workgroup

struct BwdWs {
    float *lse2;      // [B, Tq, Hq]
    int4 *rec;        // [B, Tq, Hq]: {lse2, delta (f32 bits), lo, hi - lo (>= 0)} per query row
                      // and head, what the dK/dV kernel stages for a row in one 16-byte load
    int32_t *rlo;     // [B, Tq]
    int32_t *rhi;     // [B, Tq]
    int32_t *trange;  // [B, ntiles, 4]: union lo, union hi, full lo, full hi
    int hsplit;       // dK/dV workgroups per (key block, key-value head): query heads split
    float *kvpart;    // hsplit > 1: [hsplit][2][B, Tk, Hkv, D] f32 partial dK (scaled), dV
    int32_t *kbsteps; // [B, nkb + 1]: query tiles that see each key block
    int32_t *order;   // [nwork]: dK/dV work items, the most steps first
};

template <int D>
struct BwdStrides {
    static constexpr int ROW = D + 8;  // rows read by ds_read_b128
    static constexpr int TR = D + 32;  // rows read by ds_read_b64_tr_b16
};

// The dK/dV kernels step over the queries 32 at a time, staging Q and dO tiles in slots of
// this layout.
constexpr int kDkdvStep = 32;  // queries per step
constexpr int kDkdvSlots = 3;

template <int D>
struct DkdvSlot {
    uint4 q[kDkdvStep * BwdStrides<D>::ROW / 8];
    uint4 qt[kDkdvStep * BwdStrides<D>::TR / 8];
    uint4 g[kDkdvStep * BwdStrides<D>::ROW / 8];
    uint4 gt[kDkdvStep * BwdStrides<D>::TR / 8];
    float lse2[kDkdvStep], delta[kDkdvStep];
    int32_t rlo[kDkdvStep], rhi[kDkdvStep];
};

constexpr int kDkdvRing = 8;  // schedule entries in flight (steps n - 1 .. n + 5)

// The head width 256 dK/dV launch: 2 x blocks work items (the dV and the dK passes), in the
// order of w.order.
void launch_dkdv_w4(int dtype, bool pad, int64_t blocks, const MaskInfo &m, int64_t B, int64_t Hq,
                    int64_t Hkv, float scale, const AttnStrides &sd, const uint16_t *q,
                    const uint16_t *k, const uint16_t *v, const uint16_t *d_o, const float *delta,
                    const BwdWs &w, uint16_t *dk, uint16_t *dv, hipStream_t st);

}  // namespace dm
