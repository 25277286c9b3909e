// lds_tr.hpp — BF16 tiles kept in LDS in their natural [row][column] layout
// and read as MFMA operands whose 8 consecutive k run down a column, through
// gfx950's transposing LDS read ds_read_b64_tr_b16: 16 lanes that each read
// 4 consecutive columns of rows k0 + lane/4 receive, lane i, column i of rows
// k0..k0+3.  Used where the contraction index is the row index of the
// stored tile (token-contiguous weight-gradient operands, keys of P and V
// in attention).
#pragma once
#include "ta_common.hpp"

namespace ta {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t* lds_i16x4_p;

// Byte offset of element (row r, column c) in a [rows][16 * NSTP] BF16 LDS
// tile (NSTP a power of two).  The 32-byte column units of a row are
// XOR-permuted by row bits 1..3 so that the transposing reads of rows
// {k0..k0+3, k0+8..k0+11} (one 32-lane phase) hit distinct banks; 16-byte
// chunks (c % 8 == 0) stay contiguous.
// the XOR applied to the 32-byte column unit of row r (NSTP > 1)
template <int NSTP>
__device__ __forceinline__ int tr_x(int r) {
    if constexpr (NSTP == 2) return (r >> 3) & 1;
    else if constexpr (NSTP == 4) return ((r >> 1) & 1) | (((r >> 3) & 1) << 1);
    else return (r & 3) | (((r >> 3) & 1) << 2);
}

template <int NSTP>
__device__ __forceinline__ int tr_off(int r, int c) {
    const int st = c >> 4, in = (c & 15) * 2;
    if constexpr (NSTP == 1) {
        return ((r * 32 + in) ^ (((r >> 3) & 1) << 7));
    } else {
        return r * 32 * NSTP + 32 * (st ^ tr_x<NSTP>(r)) + in;
    }
}

// MFMA operand of 16 columns [c0, c0+16) x rows [k0, k0+8) from a tile in
// tr_off layout: lane l (group g = l/16, j = l%16) reads rows k0 + 8g + j/4
// (and + 4), columns c0 + 4 (j%4) .. + 3; it receives column c0 + j of
// rows k0 + 8g .. + 7, the 16x16x32 operand layout.
template <int NSTP>
__device__ __forceinline__ bf16x8_t tr_frag(const char* __restrict__ tile, int k0, int c0, int lane) {
    const int g = lane >> 4, j = lane & 15;
    const int r = k0 + 8 * g + (j >> 2), c = c0 + 4 * (j & 3);
    i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_p)(tile + tr_off<NSTP>(r, c)));
    i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_p)(tile + tr_off<NSTP>(r + 4, c)));
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}


}  // namespace ta
