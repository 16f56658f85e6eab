// CDNA4 (gfx950) MFMA tile helpers for the chunk-WY kernels.
//
// Lane layouts (checked on MI355X):
//   v_mfma_f32_16x16x32_bf16: A[m][k] from lane m = l%16, k = 8*(l/16) + e (e < 8);
//     B[k][n] from lane n = l%16, k = 8*(l/16) + e; D[m][n] in lane n = l%16,
//     rows m = 4*(l/16) + i (i < 4).
//   v_mfma_f32_16x16x4_f32: A[m][k] lane m = l%16, k = l/16; B[k][n] lane
//     n = l%16, k = l/16; D as above.
// All bf16 operand tiles live in LDS "row-major over the reduction index"
// (X[m][r] with r contiguous), so a fragment is one 16-byte LDS read.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn2 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// 16-byte fragment: row (l%16) of a 16-row tile, reduction offset r0 + 8*(l/16).
__device__ __forceinline__ bf16x8_t frag(const uint16_t *tile, int ld, int r0) {
    const int l = lane_id();
    const uint4 v = *reinterpret_cast<const uint4 *>(tile + (l & 15) * ld + r0 + 8 * (l >> 4));
    return __builtin_bit_cast(bf16x8_t, v);
}

// acc += X[0:16, 0:R] * Y[0:16, 0:R]^T, X and Y bf16 tiles (row stride ld*).
template <int R>
__device__ __forceinline__ void mma_nt(f32x4 &acc, const uint16_t *X, int ldx, const uint16_t *Y,
                                       int ldy) {
#pragma unroll
    for (int r = 0; r < R; r += 32)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(X, ldx, r), frag(Y, ldy, r), acc, 0, 0,
                                                      0);
}

// acc += A[16x16] * B[16x16], fp32 row-major tiles in LDS (exact fp32 products).
__device__ __forceinline__ void mm16_f32(f32x4 &acc, const float *A, int lda, const float *B,
                                         int ldb) {
    const int l = lane_id();
#pragma unroll
    for (int kk = 0; kk < 16; kk += 4)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[(l & 15) * lda + kk + (l >> 4)],
                                                   B[(kk + (l >> 4)) * ldb + (l & 15)], acc, 0, 0,
                                                   0);
}

// Element (i) of a 16x16 accumulator tile: row 4*(l/16)+i, column l%16.
__device__ __forceinline__ int acc_row(int i) { return 4 * (lane_id() >> 4) + i; }
__device__ __forceinline__ int acc_col() { return lane_id() & 15; }

// Round to nearest even with the gfx950 v_cvt_pk_bf16_f32 instruction.
__device__ __forceinline__ uint16_t bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ uint32_t bf16_pack2(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t p = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, p);
}
__device__ __forceinline__ float bf16_val(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// Store an accumulator tile transposed: dst[col][row..row+3] (one 8-byte write).
__device__ __forceinline__ void store_tile_t(uint16_t *dst, int ld, const f32x4 &acc) {
    const int l = lane_id();
    *reinterpret_cast<uint2 *>(dst + (l & 15) * ld + 4 * (l >> 4)) =
        make_uint2(bf16_pack2(acc[0], acc[1]), bf16_pack2(acc[2], acc[3]));
}

// Store an accumulator tile row-major: dst[row][col] (four 2-byte writes).
__device__ __forceinline__ void store_tile_rm(uint16_t *dst, int ld, const f32x4 &acc) {
    const int l = lane_id();
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[(4 * (l >> 4) + i) * ld + (l & 15)] = bf16_bits(acc[i]);
}

// Two-term bf16 split: x ~= hi + lo with hi = bf16(x), lo = bf16(x - hi); a GEMM
// over both terms carries ~16 mantissa bits of the operand.
__device__ __forceinline__ void split_bf16(float x, uint16_t &hi, uint16_t &lo) {
    hi = bf16_bits(x);
    lo = bf16_bits(x - bf16_val(hi));
}

__device__ __forceinline__ void store_tile_t_split(uint16_t *hi_dst, uint16_t *lo_dst, int ld,
                                                   const f32x4 &acc) {
    const int l = lane_id();
    uint16_t h[4], o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) split_bf16(acc[i], h[i], o[i]);
    const int off = (l & 15) * ld + 4 * (l >> 4);
    *reinterpret_cast<uint2 *>(hi_dst + off) =
        make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
    *reinterpret_cast<uint2 *>(lo_dst + off) =
        make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16));
}

__device__ __forceinline__ void store_tile_rm_split(uint16_t *hi_dst, uint16_t *lo_dst, int ld,
                                                    const f32x4 &acc) {
    const int l = lane_id();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint16_t h, o;
        split_bf16(acc[i], h, o);
        hi_dst[(4 * (l >> 4) + i) * ld + (l & 15)] = h;
        lo_dst[(4 * (l >> 4) + i) * ld + (l & 15)] = o;
    }
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

}  // namespace gdn2
