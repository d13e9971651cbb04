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
// tests/test_gpu_mfma.py checks these layouts on the device.
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

// f32 -> 16-bit bits (bf16 round to nearest even, or f16), two at a time.
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (DT == DM_BF16) {
        uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
        ua += 0x7fffu + ((ua >> 16) & 1u);
        ub += 0x7fffu + ((ub >> 16) & 1u);
        return (ua >> 16) | (ub & 0xffff0000u);
    } else {
        union {
            _Float16 h[2];
            uint32_t u;
        } c;
        c.h[0] = (_Float16)a;
        c.h[1] = (_Float16)b;
        return c.u;
    }
}

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

// Linear block index remapped so that consecutive logical work items land on one XCD (block
// b runs on XCD b % 8): XCD x takes logical items [x * per, (x + 1) * per).
__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t nblocks) {
    const int64_t per = (nblocks + 7) / 8;
    return (b % 8) * per + b / 8;
}

}  // namespace dm
