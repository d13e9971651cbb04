// gfx950 MFMA fragments used by the attention and gated-delta-rule kernels.
//
// v_mfma_f32_32x32x16_{bf16,f16}: D[32x32] += A[32x16] B[16x32], wave64.
//   A: lane l holds row (l % 32), k = 8 * (l / 32) + [0, 8)
//   B: lane l holds col (l % 32), k = 8 * (l / 32) + [0, 8)
//   D: lane l holds col (l % 32), rows 8 * (i / 4) + 4 * (l / 32) + (i % 4), i in [0, 16)
// v_mfma_f32_16x16x32_{bf16,f16}: D[16x16] += A[16x32] B[32x16].
//   A: lane l holds row (l % 16), k = 8 * (l / 16) + [0, 8)
//   B: lane l holds col (l % 16), k = 8 * (l / 16) + [0, 8)
//   D: lane l holds col (l % 16), rows 4 * (l / 16) + i, i in [0, 4)
// Which hardware k a lane's slot is does not matter to a product as long as A and B agree; the
// kernels use that freedom to feed a product's output fragment back in as the next one's operand.
// The attention and gated-delta-rule parity tests check these layouts on the device.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dashmi.h"

namespace dm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// 8 16-bit values as raw bits, the form loads and stores move.
struct Frag8 {
    uint4 u;
};

template <int DT>
__device__ __forceinline__ f32x16_t mfma32(const Frag8 &a, const Frag8 &b, const f32x16_t &c) {
    if constexpr (DT == DM_BF16) {
        bf16x8_t av, bv;
        __builtin_memcpy(&av, &a.u, 16);
        __builtin_memcpy(&bv, &b.u, 16);
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c, 0, 0, 0);
    } else {
        f16x8_t av, bv;
        __builtin_memcpy(&av, &a.u, 16);
        __builtin_memcpy(&bv, &b.u, 16);
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, c, 0, 0, 0);
    }
}

template <int DT>
__device__ __forceinline__ f32x4_t mfma16(const Frag8 &a, const Frag8 &b, const f32x4_t &c) {
    if constexpr (DT == DM_BF16) {
        bf16x8_t av, bv;
        __builtin_memcpy(&av, &a.u, 16);
        __builtin_memcpy(&bv, &b.u, 16);
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, c, 0, 0, 0);
    } else {
        f16x8_t av, bv;
        __builtin_memcpy(&av, &a.u, 16);
        __builtin_memcpy(&bv, &b.u, 16);
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, c, 0, 0, 0);
    }
}

// f32 -> 16-bit bits, two at a time: v_cvt_pk_bf16_f32 (round to nearest even) or
// v_cvt_pk_f16_f32.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    f32x2_t x = {a, b};
    uint32_t u;
    if constexpr (DT == DM_BF16) {
        bf16x2_t y = __builtin_convertvector(x, bf16x2_t);
        __builtin_memcpy(&u, &y, 4);
    } else {
        f16x2_t y = __builtin_convertvector(x, f16x2_t);
        __builtin_memcpy(&u, &y, 4);
    }
    return u;
}

// 2^x on v_exp_f32 directly (the arguments here are finite or -inf; no range reduction).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef short s16x4_t __attribute__((ext_vector_type(4)));

// The transposed operand of a 32x32x16 product from a row-major LDS tile (rows = the product's
// k, 16-bit elements along the other index), by two ds_read_b64_tr_b16. ds_read_b64_tr_b16 hands
// lane i of each 16-lane group element i % 4 of the 8-byte row that lane 4 e + i / 4 of the group
// addressed, in slot e. With the rows addressed below, lane l receives, for index c = l % 32 of
// the operand's 32 rows/columns, the tile's elements (k0 + 8 j + 4 (l / 32) + e, c0 + c) for
// e in [0, 4) in slots 4 j + e: the k order the 32x32 products' output layout has, so a product's
// output fragment can be the other operand.
//   tile: LDS base of the row-major tile, stride: its row stride in elements.
__device__ __forceinline__ Frag8 lds_tr_frag(const uint16_t *tile, int stride, int k0, int c0,
                                             int lane) {
    const int g = lane >> 4, i = lane & 15;
    const int row = k0 + 4 * (g >> 1) + (i >> 2);
    const int colx = c0 + 16 * (g & 1) + 4 * (i & 3);
    typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
    const uint16_t *p0 = tile + row * stride + colx;
    const uint16_t *p1 = p0 + 8 * stride;
    s16x4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(p0));
    s16x4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(p1));
    Frag8 f;
    __builtin_memcpy(&f.u.x, &a, 8);
    __builtin_memcpy(&f.u.z, &b, 8);
    return f;
}

// An A or B fragment from a row-major 16-bit tile whose rows are the fragment's rows (A) or
// columns (B) and whose columns are k: rows r0 + lane % 32, k slots 16 st + 8 j + 4 h + e at
// columns k0 + 4 h + [0, 4) and k0 + 8 + 4 h + [0, 4) (the order lds_tr_frag's slots have).
__device__ __forceinline__ Frag8 row_frag(const uint16_t *t, int stride, int r0, int k0,
                                          int lane) {
    const uint16_t *p = t + (r0 + (lane & 31)) * stride + k0 + (lane >> 5) * 4;
    const uint2 lo = *(const uint2 *)p, hi = *(const uint2 *)(p + 8);
    Frag8 f;
    f.u = make_uint4(lo.x, lo.y, hi.x, hi.y);
    return f;
}

// The 32x32 product output's element i of a lane: row 8 (i / 4) + 4 (lane / 32) + i % 4 of the
// tile, column lane % 32.
__device__ __forceinline__ int crow(int i, int lane) { return (i / 4) * 8 + (lane >> 5) * 4 + (i % 4); }

template <int DT>
__device__ __forceinline__ float unpack_lo(uint32_t w) {
    if constexpr (DT == DM_BF16) {
        return __uint_as_float(w << 16);
    } else {
        union {
            uint32_t u;
            _Float16 h[2];
        } c;
        c.u = w;
        return (float)c.h[0];
    }
}

template <int DT>
__device__ __forceinline__ float unpack_hi(uint32_t w) {
    if constexpr (DT == DM_BF16) {
        return __uint_as_float(w & 0xffff0000u);
    } else {
        union {
            uint32_t u;
            _Float16 h[2];
        } c;
        c.u = w;
        return (float)c.h[1];
    }
}

// Raw buffer loads: out-of-range offsets (>= the resource's byte count) return zeros, so tile
// loads need no bounds branches. The offsets are 32-bit byte offsets from the resource's base.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(x[0], x[1], x[2], x[3]);
}
// The same with the non-temporal hint (cache policy bit 1): for data read once and streamed past,
// such as a key-value cache during decode.
__device__ __forceinline__ uint4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
    return make_uint4(x[0], x[1], x[2], x[3]);
}

// A product tile's output fragment as the B (or A) operand of a next product whose k is the
// tile's rows: k step u takes elements 8 u .. 8 u + 7.
template <int DT>
__device__ __forceinline__ Frag8 c_frag(const f32x16_t &v, int u, float f = 1.f) {
    Frag8 x;
    x.u = make_uint4(pack2<DT>(v[8 * u] * f, v[8 * u + 1] * f), pack2<DT>(v[8 * u + 2] * f, v[8 * u + 3] * f),
                     pack2<DT>(v[8 * u + 4] * f, v[8 * u + 5] * f), pack2<DT>(v[8 * u + 6] * f, v[8 * u + 7] * f));
    return x;
}

// x rounded to the dtype and back
template <int DT>
__device__ __forceinline__ float round_to(float x) {
    return unpack_lo<DT>(pack2<DT>(x, 0.f));
}

__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

__device__ __forceinline__ f32x16_t zero16() {
    f32x16_t z;
#pragma unroll
    for (int i = 0; i < 16; i++) z[i] = 0.f;
    return z;
}

// Sum over aligned groups of N lanes (N = 8, 16 or 32) by DPP moves within 16-lane rows: quad
// swaps, then the half-row mirror (lane i with 7 - i) and the row mirror (lane i with 15 - i)
// pair lanes from the other half each time, so every lane ends with its group's sum.
template <int N>
__device__ __forceinline__ float group_sum(float t) {
#define DM_DPP(x, ctrl) \
    __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), ctrl, 0xf, 0xf, false))
    t += DM_DPP(t, 0xB1);   // quad_perm [1, 0, 3, 2]
    t += DM_DPP(t, 0x4E);   // quad_perm [2, 3, 0, 1]
    t += DM_DPP(t, 0x141);  // row_half_mirror
    if constexpr (N >= 16) t += DM_DPP(t, 0x140);  // row_mirror
#undef DM_DPP
    if constexpr (N >= 32) t += __shfl_xor(t, 16, 64);
    return t;
}

}  // namespace dm
