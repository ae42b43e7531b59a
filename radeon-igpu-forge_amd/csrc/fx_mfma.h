// bf16 MFMA operand helpers shared by the attention and GEMM kernels (gfx950).
//
// v_mfma_f32_32x32x16_bf16, wave64:
//   A (32 x 16): lane l supplies row l%32, k = 8*(l/32) + 0..7
//   B (16 x 32): lane l supplies column l%32, k = 8*(l/32) + 0..7
//   C (32 x 32): lane l holds column l%32, rows 8*(i/4) + 4*(l/32) + i%4, i = 0..15
// An operand whose K dimension runs down the rows of a row-major LDS tile is read with
// ds_read_b64_tr_b16: within a group of 16 lanes, lane s points at row k0 + s/4,
// column m0 + 4*(s%4) and lane i receives column m0 + i of rows k0..k0+3; two such
// reads give the 8 K-values, at the permuted positions j < 4 -> 4*g + j,
// j >= 4 -> 8 + 4*g + j - 4 (g = l/32).  Two operands read this way see the same
// permutation, so their product is the plain contraction.
#pragma once

#include "fx_device.h"

namespace fx {

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x4 lds_tr16(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
        (lds_bf16x4*)(__attribute__((address_space(3))) void*)(p));
}

__device__ __forceinline__ bf16x8 cat8(const bf16x4& lo, const bf16x4& hi) {
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Operand whose K dimension runs down the rows of a row-major LDS tile with row stride
// `ld` (elements): K rows k0.. (k0 the 16-row chunk base), columns m0 + 0..31
// (lane l -> column m0 + l%32).
__device__ __forceinline__ bf16x8 lds_op_t(const uint16_t* tile, int ld, int k0, int m0, int lane) {
    const int grp = lane >> 4, s = lane & 15;
    const int row = k0 + 4 * (grp >> 1) + (s >> 2);
    const int col = m0 + 16 * (grp & 1) + 4 * (s & 3);
    const uint16_t* p = tile + row * ld + col;
    return cat8(lds_tr16(p), lds_tr16(p + 8 * ld));
}

// Operand whose K dimension runs along a row: lane l reads 8 contiguous elements of
// row r0 + l%32 starting at column c0 + 8*(l/32).
__device__ __forceinline__ bf16x8 lds_op_row(const uint16_t* tile, int ld, int r0, int c0, int lane) {
    return *reinterpret_cast<const bf16x8*>(tile + (r0 + (lane & 31)) * ld + c0 + 8 * (lane >> 5));
}

}  // namespace fx
