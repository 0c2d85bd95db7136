// Helpers shared by the prefill attention kernels (gfx950).
#pragma once

#include "common.hpp"

namespace sl8 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

typedef __attribute__((address_space(1))) const void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

// Direct global -> LDS copy: lane i of the wave writes `bytes` at lds + i*bytes.
__device__ __forceinline__ void dma16_to_lds(const void* g, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((gptr_t)g, (lptr_t)lds_wave_base, 16, 0, 0);
}
__device__ __forceinline__ void dma4_to_lds(const void* g, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((gptr_t)g, (lptr_t)lds_wave_base, 4, 0, 0);
}
__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// Keeps the computation of `x` ahead of this point: an empty volatile asm
// that reads it, which neither the IR passes nor the machine scheduler move
// across a scheduling barrier (they may otherwise sink pure arithmetic to its
// first real use, out of the slice it was placed in).
template <typename T>
__device__ __forceinline__ void pin_vgpr(const T& x) {
  asm volatile("" ::"v"(x));
}

// max(x, x of lane ^ 32) in every lane of the wave: one v_permlane32_swap
// (lanes 0-31 receive lanes 32-63 and back; a VALU op, no LDS round trip)
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// blockIdx.x -> (b*Hq + h, slot). Slots are issued in increasing order, so
// callers put their heaviest work in slot 0. With xcd_map, workgroup ids are
// dealt so that each KV head's query heads stay on one XCD (id % 8 is the
// XCD) and share its L2:
//   B*Hkv a multiple of 8: XCD x serves KV heads x, x+8, ...;
//   B*Hkv dividing 8 (rep = 8 / (B*Hkv) XCDs per KV head): XCD x serves KV
//   head x % (B*Hkv), taking every rep-th (slot, head) unit of it.
// xcd_mode(): 1 / 2 for those cases, 0 = plain order (host-side choice).
inline int xcd_mode(long long nbkv, long long gsz, long long nslot) {
  if (nbkv % 8 == 0) return 1;
  if (8 % nbkv == 0 && (gsz * nslot) % (8 / nbkv) == 0) return 2;
  return 0;
}

__device__ __forceinline__ void attn_block_coords(int Hq, int Hkv, int nslot, int xcd_map,
                                                  int& bh, int& slot) {
  const int id = blockIdx.x;
  const int total = gridDim.x;
  const int gsz = Hq / Hkv;
  if (xcd_map == 1) {
    const int nbkv = total / (nslot * gsz);  // B * Hkv
    const int xcd = id & 7, k = id >> 3;
    const int per_slot = (nbkv / 8) * gsz;
    const int r = k / per_slot;
    const int rem = k % per_slot;
    const int bkv = xcd + 8 * (rem / gsz);
    const int j = rem % gsz;
    const int b = bkv / Hkv, kvh = bkv % Hkv;
    bh = b * Hq + kvh * gsz + j;
    slot = r;
  } else if (xcd_map == 2) {
    const int nbkv = total / (nslot * gsz);  // divides 8
    const int rep = 8 / nbkv;
    const int xcd = id & 7, k = id >> 3;
    const int bkv = xcd % nbkv, sub = xcd / nbkv;
    const int u = k * rep + sub;             // (slot, head) unit of this KV head
    const int b = bkv / Hkv, kvh = bkv % Hkv;
    bh = b * Hq + kvh * gsz + u % gsz;
    slot = u / gsz;
  } else {
    const int nbh = total / nslot;
    slot = id / nbh;
    bh = id % nbh;
  }
}

}  // namespace sl8
