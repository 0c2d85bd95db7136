// Shared helpers for the gfx950 kernels and the C-ABI entry points.
//
// Every entry point returns an sl8 status code (0 = ok) and records a message
// readable through sl8_last_error(); nothing throws across the C boundary.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bfloat16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "../../include/superl8_hip.h"

namespace sl8 {

// Last-error slot (per host thread).
void set_error(const char* fmt, ...);
void clear_error();

#define SL8_CHECK_ARG(cond, ...)                 \
  do {                                           \
    if (!(cond)) {                               \
      ::sl8::set_error(__VA_ARGS__);             \
      return SL8_ERR_INVALID;                    \
    }                                            \
  } while (0)

#define SL8_CHECK_LAUNCH(what)                                                  \
  do {                                                                          \
    hipError_t e_ = hipGetLastError();                                          \
    if (e_ != hipSuccess) {                                                     \
      ::sl8::set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e_)); \
      return SL8_ERR_LAUNCH;                                                    \
    }                                                                           \
  } while (0)

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ---- scalar conversions (round-to-nearest-even everywhere) ----
__device__ __forceinline__ float ld_f(const __half* p) { return __half2float(*p); }
__device__ __forceinline__ float ld_f(const hip_bfloat16* p) { return static_cast<float>(*p); }
__device__ __forceinline__ float ld_f(const float* p) { return *p; }

__device__ __forceinline__ float h2f(uint16_t bits) {
  return __half2float(__ushort_as_half(bits));
}
__device__ __forceinline__ float bf2f(uint16_t bits) {
  return __uint_as_float(static_cast<uint32_t>(bits) << 16);
}
// fp32 -> bf16 bits, round-to-nearest-even (NaN kept quiet).
__device__ __forceinline__ uint16_t f2bf_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ uint16_t f2h_bits(float f) { return __half_as_ushort(__float2half_rn(f)); }

// Typed store of one fp32 value as fp16 / bf16 / fp32.
template <int DT> __device__ __forceinline__ void st_out(void* base, int64_t i, float v);
template <> __device__ __forceinline__ void st_out<SL8_DTYPE_F16>(void* b, int64_t i, float v) {
  reinterpret_cast<uint16_t*>(b)[i] = f2h_bits(v);
}
template <> __device__ __forceinline__ void st_out<SL8_DTYPE_BF16>(void* b, int64_t i, float v) {
  reinterpret_cast<uint16_t*>(b)[i] = f2bf_bits(v);
}
template <> __device__ __forceinline__ void st_out<SL8_DTYPE_F32>(void* b, int64_t i, float v) {
  reinterpret_cast<float*>(b)[i] = v;
}

// 16-bit storage element -> fp32 for fp16 / bf16.
template <int DT> __device__ __forceinline__ float u16_to_f(uint16_t b);
template <> __device__ __forceinline__ float u16_to_f<SL8_DTYPE_F16>(uint16_t b) { return h2f(b); }
template <> __device__ __forceinline__ float u16_to_f<SL8_DTYPE_BF16>(uint16_t b) { return bf2f(b); }

// Wave64 reductions (DPP/bpermute chosen by the compiler from __shfl_xor).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Buffer-resource copies to LDS: a raw buffer of `bytes` bytes at `base`
// (stride 0; the gfx9-family format dword). The per-lane byte offset stays in a
// VGPR and the per-tile advance goes in the scalar offset, so a tile copy costs
// no vector address arithmetic; offsets at or past `bytes` read as zero.
typedef __amdgpu_buffer_rsrc_t brsrc_t;
__device__ __forceinline__ brsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void buf16_to_lds(brsrc_t r, void* lds_wave_base, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_wave_base, 16,
                                           voff, soff, 0, 0);
}
__device__ __forceinline__ void buf4_to_lds(brsrc_t r, void* lds_wave_base, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_wave_base, 4,
                                           voff, soff, 0, 0);
}

// CUs of the current device (cached per device)
inline int cu_count() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus[dev] = 256;
  return cus[dev] > 0 ? cus[dev] : 256;
}

}  // namespace sl8
