// Shared pieces of the GGUF k-quant kernels (Q4_K, Q5_K, Q6_K).
#pragma once

#include "common.hpp"

#ifndef SL8_KQ_XCD
#define SL8_KQ_XCD 1
#endif

namespace sl8 {

// Packed 6-bit sub-scales / mins of a Q4_K / Q5_K super-block (4 per dword,
// byte j % 4), unpacked from the 12-byte get_scale_min_k4 layout.
struct ScMin {
  uint32_t sc_lo, sc_hi, mn_lo, mn_hi;
};
__device__ __forceinline__ ScMin unpack_scmin(uint32_t s0, uint32_t s1, uint32_t s2) {
  ScMin r;
  r.sc_lo = s0 & 0x3F3F3F3Fu;
  r.mn_lo = s1 & 0x3F3F3F3Fu;
  r.sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
  r.mn_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
  return r;
}
// Tile order o -> (column tile ct, row tile rt) of the k-quant tile GEMMs.
// xcd_m > 0 (the number of row tiles; used when the column-tile count is a
// multiple of 8): workgroup o runs on XCD o % 8, and the xcd_m row tiles of
// one weight column tile are consecutive workgroups of the same XCD, so the
// column's weights come from HBM into that XCD's L2 once and are re-read
// from there by the other row tiles running beside it. xcd_m = 0: row-major.
__device__ __forceinline__ void kq_tile_coords(int o, int nt_x, int xcd_m, int& ct, int& rt) {
  if (xcd_m > 0) {
    const int k = o >> 3;
    ct = (o & 7) + 8 * (k / xcd_m);
    rt = k % xcd_m;
  } else {
    ct = o % nt_x;
    rt = o / nt_x;
  }
}
__device__ __forceinline__ int byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFF; }

// Four byte lanes times one small factor, for products that stay below 256
// per byte (no carries between bytes): one packed 16-bit multiply
// (v_pk_mul_lo_u16, full rate) instead of a 32-bit integer multiply (quarter
// rate); each 16-bit half holds two bytes and its product stays below 2^16.
__device__ __forceinline__ uint32_t mul_bytes(uint32_t bytes, uint32_t f) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  const u16x2 a = __builtin_bit_cast(u16x2, bytes);
  const u16x2 b = {(unsigned short)f, (unsigned short)f};
  return __builtin_bit_cast(uint32_t, a * b);
}

// Q5_K decode GEMV for M <= 2 on the Q4_K M <= 2 kernel (gemm_q4k.hip)
void launch_gemv_q5k_small(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                           int M, int N, int K, hipStream_t st);
// Q5_K decode GEMV for 3 <= M <= 16 on the int8 MFMA (gemm_q4k.hip)
void launch_gemv_q5k_mfma(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                          int M, int N, int K, hipStream_t st);

typedef __attribute__((address_space(1))) const void* kq_gptr_t;
typedef __attribute__((address_space(3))) void* kq_lptr_t;

}  // namespace sl8
