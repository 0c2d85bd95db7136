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

// blockIdx.x -> (b*Hq + h, slot). Slots are issued in increasing order, so
// callers put their heaviest work in slot 0. With xcd_map (B*Hkv a multiple
// of 8) workgroup ids are dealt so that XCD x (= id % 8) only serves KV heads
// x, x+8, ...: the query heads sharing a KV head then share that XCD's L2.
__device__ __forceinline__ void attn_block_coords(int Hq, int Hkv, int nslot, bool xcd_map,
                                                  int& bh, int& slot) {
  const int id = blockIdx.x;
  const int total = gridDim.x;
  const int gsz = Hq / Hkv;
  if (xcd_map) {
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
  } else {
    const int nbh = total / nslot;
    slot = id / nbh;
    bh = id % nbh;
  }
}

}  // namespace sl8
