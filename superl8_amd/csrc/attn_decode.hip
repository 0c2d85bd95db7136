// Split-KV decode attention (M = 1) for gfx950: int8 K with per-token fp32
// scales, fp16 V, exp2-domain online softmax, log-sum-exp merge of splits.
//
// Semantics follow the reference (csrc/include/attn_decode.cuh:47-132,430-466):
//   split s owns keys [s*per, min(N, (s+1)*per)), per = ceil(N / num_splits);
//   logit = ((float)<q_i8, k_i8> * q_scale) * k_scale[n]   (exp2 domain)
//   partial (O[D], m, l) per (split, query head); an empty split writes
//   m = -1e30, l = 0, O = 0; combine: O = sum O_s 2^(m_s-M) / sum l_s 2^(m_s-M).
//
// MI355X design (the path is HBM-bound, ~1.6 GB per call at the B16/N32k shape):
//   * one workgroup per (split, batch, KV head, query-head chunk): the G query
//     heads of a GQA group share every K/V byte read, so each KV byte is
//     fetched from HBM once, not once per query head;
//   * QK: lane = key, the whole int8 K row is loaded as 16-byte vectors and
//     dotted with v_dot4_i32_i8 against Q broadcast from LDS;
//   * PV: lane = (8 consecutive channels, key phase); V rows arrive as
//     16-byte loads (a wave reads D*2*64/(D/8) contiguous bytes per step);
//     P is handed over through LDS;
//   * 4 waves take interleaved 64-key tiles with private online-softmax
//     state and are merged by LSE in LDS at the end (fixed order, so results
//     are deterministic).

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.hpp"

namespace sl8 {
namespace {

constexpr int DEC_THREADS = 256;
constexpr int DEC_WAVES = 4;
constexpr int DEC_TILE = 64;
constexpr float DEC_NEG_INF = -1e30f;
constexpr int DEC_MAX_SPLITS = 256;
#ifndef SL8_DEC_PAIR
#define SL8_DEC_PAIR 1
#endif
constexpr bool DEC_PAIR = SL8_DEC_PAIR;  // int8-V PV: two keys per v_dot2 (see decode_wave_kernel)
// query heads (waves) per merge workgroup: one, so config 3's 512 heads spread
// over all CUs (4 per workgroup measured ~1 us slower per decode call)
constexpr int CMB_WAVES = 1;
#ifndef SL8_DEC_PV4
#define SL8_DEC_PV4 1
#endif

template <int D, int G>
struct DecSmem {
  int q[G][D / 4];                 // int8 Q, packed
  float qs[G];
  float p[DEC_WAVES][DEC_TILE][G];  // per-wave probabilities of the current tile
  float m[DEC_WAVES][G];
  float l[DEC_WAVES][G];
  float o[DEC_WAVES][G][D];
};

// VI8: V is the int8 cache [B,Hkv,N,D] with per-channel scale vsc [B,Hkv,D]
// (reference attn_decode.cuh:141-224), folded into the partial O.
// PG (paged, reference attn_paged_decode.cuh:126-262): K/V int8 caches
// [num_blocks,Hkv,bs,D] with per-token scales [num_blocks,Hkv,bs] for both;
// key n of sequence b is row (bt[b][n / bs] * Hkv + kvh) * bs + n % bs; the
// sequence has ctx[b] keys and the splits are sized on n_len (the launch's
// maximum); the per-token V scale multiplies p inside the key sum.
struct PagedArgs {
  const int32_t* bt;   // [B, maxb] physical block per logical block
  const int32_t* ctx;  // [B] keys per sequence
  int maxb, bs;
  int bs_sh;           // log2(bs) (streaming kernels: bs a power of two; K8V3: -1 if not)
  int cache_rows;      // num_blocks * Hkv * bs (streaming kernel, block-aligned tiles)
};
// block-table entries of one split staged in LDS by the streaming paged kernel
constexpr int DEC_BT_MAX = 1024;

// Per-token K scale of key row r: fp32 (the reference contract) or, with
// KS16, fp16 (half the scale bytes; BASELINE config 3's cache format).
template <bool KS16>
__device__ __forceinline__ float load_ks(const void* base, int64_t r) {
  if constexpr (KS16) return h2f(static_cast<const uint16_t*>(base)[r]);
  else return static_cast<const float*>(base)[r];
}

template <int D, int G, bool VI8, bool PG, bool KS16 = false>
__global__ void __launch_bounds__(DEC_THREADS)
decode_split_kernel(const int8_t* __restrict__ q, const float* __restrict__ q_scale,
                    const int8_t* __restrict__ k, const void* __restrict__ k_scale,
                    const void* __restrict__ v, const float* __restrict__ vsc,
                    float* __restrict__ o_part,
                    float* __restrict__ m_part, float* __restrict__ l_part, int n_len,
                    int n_splits, int h_q, int h_kv, int gsz, int bhq, const PagedArgs pg) {
  static_assert(!PG || VI8, "the paged cache holds int8 V");
  constexpr int D4 = D / 4;
  constexpr int DG = D / 8;           // 8-channel groups
  constexpr int KPH = 64 / DG;        // key phases in the PV lane map
  constexpr int KPL = DEC_TILE / KPH; // keys per lane per tile in PV
  __shared__ DecSmem<D, G> sm;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int split = blockIdx.x;
  const int bkv = blockIdx.y;  // b * h_kv + kvh
  const int b = bkv / h_kv, kvh = bkv % h_kv;
  const int j0 = blockIdx.z * G;  // first head of this chunk within the group
  const int ng = min(G, gsz - j0);

  // stage Q of the chunk's heads
  for (int i = tid; i < G * D4; i += DEC_THREADS) {
    const int g = i / D4, c = i % D4;
    int val = 0;
    if (g < ng) {
      const int64_t hq = (int64_t)b * h_q + kvh * gsz + j0 + g;
      val = reinterpret_cast<const int*>(q + hq * D)[c];
    }
    sm.q[g][c] = val;
  }
  if (tid < G) {
    const int64_t hq = (int64_t)b * h_q + kvh * gsz + j0 + tid;
    sm.qs[tid] = tid < ng ? q_scale[hq] : 0.f;
  }
  __syncthreads();

  const int per = (n_len + n_splits - 1) / n_splits;
  const int n0 = split * per;
  // paged: a context length above max_context_len (n_len) is read as
  // max_context_len, so no block-table entry past the table's capacity is used
  const int n1 = min(PG ? min(pg.ctx[b], n_len) : n_len, n0 + per);
  // cache row of key n (contiguous: relative to this (batch, KV head))
  const int32_t* btb = PG ? pg.bt + (int64_t)b * pg.maxb : nullptr;
  auto krow = [&](int n) -> int64_t {
    if constexpr (PG) return ((int64_t)btb[n / pg.bs] * h_kv + kvh) * pg.bs + n % pg.bs;
    else return n;
  };
  const int8_t* kb = k + (PG ? 0 : (int64_t)bkv * n_len * D);
  const void* ksb = static_cast<const uint8_t*>(k_scale) +
                    (PG ? 0 : (int64_t)bkv * n_len * (KS16 ? 2 : 4));
  constexpr int VES = VI8 ? 1 : 2;  // V element bytes
  const uint8_t* vb = static_cast<const uint8_t*>(v) + (PG ? 0 : (int64_t)bkv * n_len * D * VES);

  float m_run[G], l_lane[G], oacc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_lane[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) oacc[g][e] = 0.f;
  }
  const int dg = lane % DG, kph = lane / DG;

  for (int t0 = n0 + wave * DEC_TILE; t0 < n1; t0 += DEC_WAVES * DEC_TILE) {
    // ---- logits: lane = key ----
    const int n = t0 + lane;
    const bool valid = n < n1;
    float s[G];
    {
      int4 kr[D / 16];
      const int64_t kr_row = krow(valid ? n : n0);
      const int4* kp = reinterpret_cast<const int4*>(kb + kr_row * D);
#pragma unroll
      for (int c = 0; c < D / 16; ++c) kr[c] = kp[c];
      const float ks = valid ? load_ks<KS16>(ksb, kr_row) : 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        int acc = 0;
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          const int4 qv = *reinterpret_cast<const int4*>(&sm.q[g][4 * c]);
          acc = __builtin_amdgcn_sdot4(qv.x, kr[c].x, acc, false);
          acc = __builtin_amdgcn_sdot4(qv.y, kr[c].y, acc, false);
          acc = __builtin_amdgcn_sdot4(qv.z, kr[c].z, acc, false);
          acc = __builtin_amdgcn_sdot4(qv.w, kr[c].w, acc, false);
        }
        s[g] = valid ? ((float)acc * sm.qs[g]) * ks : -INFINITY;
      }
    }
    // ---- online softmax (wave-uniform running max per head) ----
    float resc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mt = wave_max(s[g]);
      const float mn = fmaxf(m_run[g], mt);
      resc[g] = exp2f(m_run[g] - mn);  // m_run = -inf -> 0 (state is all zero then)
      m_run[g] = mn;
      const float p = exp2f(s[g] - mn);
      l_lane[g] = l_lane[g] * resc[g] + p;
      sm.p[wave][lane][g] = p;
    }
    // the wave's own region of LDS: make the writes visible to the other lanes
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- PV: lane = (channel group dg, key phase kph) ----
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) oacc[g][e] *= resc[g];
#pragma unroll 4
    for (int i = 0; i < KPL; ++i) {
      const int kk = kph + i * KPH;
      const int nn = t0 + kk;
      if (nn < n1) {
        float vf[8];
        const int64_t vr = krow(nn);
        const float pvs = PG ? vsc[vr] : 1.f;  // per-token V scale (paged)
        if constexpr (VI8) {
          const uint2 vv = *reinterpret_cast<const uint2*>(vb + vr * D + dg * 8);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            vf[e] = (float)(int8_t)(vv.x >> (8 * e));
            vf[4 + e] = (float)(int8_t)(vv.y >> (8 * e));
          }
        } else {
          const uint4 vv = *reinterpret_cast<const uint4*>(vb + (vr * D + dg * 8) * 2);
          vf[0] = h2f(vv.x & 0xFFFF); vf[1] = h2f(vv.x >> 16);
          vf[2] = h2f(vv.y & 0xFFFF); vf[3] = h2f(vv.y >> 16);
          vf[4] = h2f(vv.z & 0xFFFF); vf[5] = h2f(vv.z >> 16);
          vf[6] = h2f(vv.w & 0xFFFF); vf[7] = h2f(vv.w >> 16);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float p = sm.p[wave][kk][g] * pvs;
#pragma unroll
          for (int e = 0; e < 8; ++e) oacc[g][e] = fmaf(p, vf[e], oacc[g][e]);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // p region reused by the next tile
  }

  // ---- reduce lanes of the wave: l over all lanes, O over key phases ----
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float lw = wave_sum(l_lane[g]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = oacc[g][e];
#pragma unroll
      for (int o = DG; o < 64; o <<= 1) x += __shfl_xor(x, o, 64);
      oacc[g][e] = x;
    }
    if (lane == 0) {
      sm.m[wave][g] = m_run[g];
      sm.l[wave][g] = lw;
    }
    if (kph == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sm.o[wave][g][dg * 8 + e] = oacc[g][e];
    }
  }
  __syncthreads();

  // ---- merge the 4 waves (fixed order) and write the split partial ----
  for (int i = tid; i < G * D; i += DEC_THREADS) {
    const int g = i / D, d = i % D;
    if (g >= ng) continue;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < DEC_WAVES; ++w) mm = fmaxf(mm, sm.m[w][g]);
    float acc = 0.f, den = 0.f;
    if (mm != -INFINITY) {
#pragma unroll
      for (int w = 0; w < DEC_WAVES; ++w) {
        const float wt = exp2f(sm.m[w][g] - mm);
        acc += sm.o[w][g][d] * wt;
        den += sm.l[w][g] * wt;
      }
    }
    const int64_t hq = (int64_t)b * h_q + kvh * gsz + j0 + g;
    const int64_t row = (int64_t)split * bhq + hq;
    o_part[row * D + d] = (VI8 && !PG) ? acc * vsc[(int64_t)bkv * D + d] : acc;
    if (d == 0) {
      m_part[row] = (mm == -INFINITY) ? DEC_NEG_INF : mm;
      l_part[row] = den;
    }
  }
}

// Cross-split LSE merge (reference attn_decode.cuh:430-466):
//   gm = max_s m_s, out = sum_s o_s 2^(m_s - gm) / sum_s l_s 2^(m_s - gm),
// empty splits (m_s = DEC_NEG_INF) contributing nothing. One wave per query
// head (CMB_WAVES per workgroup): the lanes hold D / 64 channels each and every partial load of the head is issued
// before any is used; the split weights 2^(m_s - gm) are formed once per
// split by the lane that loaded m_s and broadcast, and the sums run over the
// splits in index order (deterministic).
template <int D>
__global__ void __launch_bounds__(CMB_WAVES * 64)
decode_combine_wave_kernel(const float* __restrict__ o_part, const float* __restrict__ m_part,
                           const float* __restrict__ l_part, uint16_t* __restrict__ out,
                           int n_splits, int bhq) {
  // D = 32: one channel per lane, lanes 32..63 idle
  constexpr int CPL = D >= 64 ? D / 64 : 1;
  const int lane = threadIdx.x & 63;
  const int64_t hq = (int64_t)blockIdx.x * CMB_WAVES + (threadIdx.x >> 6);
  if (hq >= bhq) return;  // wave-uniform
  constexpr int SCH = 16;  // splits whose partials are in flight together
  const bool act = CPL * lane < D;
  const float* ob = o_part + hq * D + (act ? CPL * lane : 0);
  // partial O of splits s0 .. s0 + SCH - 1 (clamped to the last split)
  auto load_o = [&](int s0, float (&ov)[SCH][CPL]) {
#pragma unroll
    for (int i = 0; i < SCH; ++i) {
      const int sp = min(s0 + i, n_splits - 1);
      const float* src = ob + (int64_t)sp * bhq * D;
      if constexpr (CPL == 4) {
        const float4 v4 = *reinterpret_cast<const float4*>(src);
        ov[i][0] = v4.x; ov[i][1] = v4.y; ov[i][2] = v4.z; ov[i][3] = v4.w;
      } else if constexpr (CPL == 2) {
        const float2 v2 = *reinterpret_cast<const float2*>(src);
        ov[i][0] = v2.x; ov[i][1] = v2.y;
      } else {
        ov[i][0] = *src;
      }
    }
  };
  // the first SCH splits' O is loaded together with every m and l (one round trip
  // for n_splits <= SCH)
  float ov[SCH][CPL];
  load_o(0, ov);
  // m, l of splits lane, lane + 64, ... (n_splits <= DEC_MAX_SPLITS = 4 x 64)
  float ms[DEC_MAX_SPLITS / 64], ls[DEC_MAX_SPLITS / 64];
  float gm = DEC_NEG_INF;
#pragma unroll
  for (int c = 0; c < DEC_MAX_SPLITS / 64; ++c) {
    const int sp = c * 64 + lane;
    ms[c] = sp < n_splits ? m_part[(int64_t)sp * bhq + hq] : DEC_NEG_INF;
    ls[c] = sp < n_splits ? l_part[(int64_t)sp * bhq + hq] : 0.f;
    gm = fmaxf(gm, ms[c]);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) gm = fmaxf(gm, __shfl_xor(gm, o, 64));
  float wt[DEC_MAX_SPLITS / 64];
  float den = 0.f;
#pragma unroll
  for (int c = 0; c < DEC_MAX_SPLITS / 64; ++c) {
    wt[c] = (ms[c] == DEC_NEG_INF) ? 0.f : exp2f(ms[c] - gm);
    den += ls[c] * wt[c];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) den += __shfl_xor(den, o, 64);
  float acc[CPL];
#pragma unroll
  for (int e = 0; e < CPL; ++e) acc[e] = 0.f;
  for (int s0 = 0; s0 < n_splits; s0 += SCH) {
    if (s0) load_o(s0, ov);
    // weights of splits s0 .. s0 + SCH - 1 live in register wt[s0 / 64] of lanes (s0 % 64) ..
    const int c = s0 >> 6;
    const float wc = c == 0 ? wt[0] : (c == 1 ? wt[1] : (c == 2 ? wt[2] : wt[3]));
#pragma unroll
    for (int i = 0; i < SCH; ++i) {
      const int sp = s0 + i;
      if (sp < n_splits) {  // wave-uniform
        const float w = __shfl(wc, sp & 63, 64);
#pragma unroll
        for (int e = 0; e < CPL; ++e) acc[e] += ov[i][e] * w;
      }
    }
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
#pragma unroll
  for (int e = 0; e < CPL; ++e)
    if (act) out[hq * D + CPL * lane + e] = f2h_bits(den > 0.f ? acc[e] * inv : 0.f);
}

template <typename... A>
void launch_combine(int D, int bhq, hipStream_t st, A... args) {
  const dim3 g((unsigned)((bhq + CMB_WAVES - 1) / CMB_WAVES));
  const dim3 b(CMB_WAVES * 64);
  if (D == 32) decode_combine_wave_kernel<32><<<g, b, 0, st>>>(args...);
  else if (D == 64) decode_combine_wave_kernel<64><<<g, b, 0, st>>>(args...);
  else if (D == 128) decode_combine_wave_kernel<128><<<g, b, 0, st>>>(args...);
  else decode_combine_wave_kernel<256><<<g, b, 0, st>>>(args...);
}

// ---------------------------------------------------------------------------
// Streaming variant for GQA groups of 2 (D = 128), 4 or 8 query heads (the serving
// shapes). Each wave is an independent stream over every 4th T-key tile of
// the split: it copies its tiles HBM -> LDS with global_load_lds into a
// private NB-stage ring and waits only on its own copies (no workgroup
// barrier inside the loop), so loads of later tiles stay in flight while the
// current tile is computed. Lane roles inside a wave (KL = 64 / GS lanes per
// query head):
//   * QK:  lane = (head h, key kl): v_dot4 over the int8 K row read from LDS
//          (rows XOR-swizzled by 16-byte chunk, so the KL rows read together
//          hit distinct banks) against that head's Q held in registers;
//   * softmax: tile max / sums reduce over the KL lanes of a head;
//   * PV:  lane = (head h, channel slice kl): CPL = D / KL channels, fp16 V
//          converted inside v_fma_mix against P broadcast from LDS.
// The 4 waves' states are merged by LSE in LDS at the end (fixed order).
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(1))) const void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

// Value of lane (lane & ~(G-1)) + r, for G = 8, 16 or 32 (r a constant):
// ds_swizzle bit mode within 32 lanes, lane' = (lane & and_mask) | or_mask.
// It moves registers only (no LDS memory access), so it never waits on
// LDS copies in flight.
template <int G, int R>
__device__ __forceinline__ float lane_bcast(float x) {
  static_assert(G == 8 || G == 16 || G == 32, "group width");
  static_assert(R >= 0 && R < G, "source lane");
  constexpr int AND = 31 & ~(G - 1);
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), AND | (R << 5)));
}

// f(std::integral_constant<int, I>) for I = 0 .. N-1, fully unrolled.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

template <int D, int GS, bool VI8 = false, bool PG = false>
struct WaveCfg {
  static constexpr int KL = 64 / GS;                  // lanes (keys) per head per sub-block
  static constexpr int SUB = KL >= 16 ? 1 : 16 / KL;  // sub-blocks per tile
  static constexpr int T = KL * SUB;                  // keys per tile
  static constexpr int CPL = D / KL;                  // PV channels per lane
  static constexpr int KC = D / 16;                   // 16-byte chunks per K row
  // K rows (D bytes) are read 16 rows per 16 lanes; LDS has 64 four-byte
  // banks (256 B), so chunks are XOR-swizzled with the row index above the
  // rows that share one 256-byte bank line.
  static constexpr int KSW = KC - 1;
  static constexpr int KSH = D == 64 ? 2 : (D == 128 ? 1 : 0);
  static constexpr int VRB = VI8 ? D : 2 * D;  // bytes per V row
  static constexpr int KBYTES = T * D, VBYTES = T * VRB;
  static constexpr int KDMA = KBYTES / 1024, VDMA = VBYTES / 1024;  // 1 KiB copies per wave
  // + k_scale (64 floats), + the per-token v_scale of a paged cache
  static constexpr int STAGE = KBYTES + VBYTES + (PG ? 512 : 256);
  static_assert(KDMA >= 1 && KBYTES % 1024 == 0, "tile copy granularity");
  static_assert(CPL % 8 == 0 || CPL == 4, "PV slice: 4 or a multiple of 8 channels");
};

// PG: paged int8 cache (see PagedArgs): the split's block-table entries are
// staged in LDS, every copy lane maps its key to a physical row, and the
// per-token V scale multiplies p before it is broadcast to the PV lanes.
// PGA (paged, block-aligned tiles): every T-key tile lies inside one cache
// block, so a tile's physical rows are one uniform base plus the lane's fixed
// offset and its copies go through buffer resources like the contiguous ones.
template <int D, int GS, int NB, bool VI8, bool PG, bool KS16 = false, bool PGA = false>
__global__ void __launch_bounds__(DEC_THREADS, (SL8_DEC_PV4 && VI8 && DEC_PAIR && D == 128 && GS == 4) ? 3 : 1)
decode_wave_kernel(const int8_t* __restrict__ q, const float* __restrict__ q_scale,
                   const int8_t* __restrict__ k, const void* __restrict__ k_scale,
                   const void* __restrict__ v, const float* __restrict__ vsc,
                   float* __restrict__ o_part,
                   float* __restrict__ m_part, float* __restrict__ l_part, int n_len,
                   int n_splits, int h_q, int h_kv, int bhq, const PagedArgs pg) {
  static_assert(!PG || VI8, "the paged cache holds int8 V");
  using C = WaveCfg<D, GS, VI8, PG>;
  constexpr int KL = C::KL, SUB = C::SUB, T = C::T, CPL = C::CPL, KC = C::KC, KSW = C::KSW;
  constexpr int KSH = C::KSH;
  constexpr int STAGE = C::STAGE;
  static_assert(NB >= 2 && NB <= 4, "ring depth");
  // One LDS object per ring stage: the compiler then knows a copy into one
  // stage never aliases reads of another and inserts no early vmcnt waits.
  __shared__ __attribute__((aligned(16))) int8_t st0[DEC_WAVES * STAGE];
  __shared__ __attribute__((aligned(16))) int8_t st1[DEC_WAVES * STAGE];
  __shared__ __attribute__((aligned(16))) int8_t st2[NB > 2 ? DEC_WAVES * STAGE : 16];
  __shared__ __attribute__((aligned(16))) int8_t st3[NB > 3 ? DEC_WAVES * STAGE : 16];
  static_assert(DEC_WAVES * STAGE >= DEC_WAVES * GS * (D + 2) * 4, "merge area fits stage 0");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  auto stage = [&](int u) -> int8_t* {
    int8_t* s = u == 0 ? st0 : (u == 1 ? st1 : (u == 2 ? st2 : st3));
    return s + wave * STAGE;
  };

  const int split = blockIdx.x;
  const int bkv = blockIdx.y;
  const int b = bkv / h_kv, kvh = bkv % h_kv;
  const int per = (n_len + n_splits - 1) / n_splits;
  const int n0 = split * per;
  // paged: a context length above max_context_len (n_len) is read as
  // max_context_len, so no block-table entry past the table's capacity is used
  const int n1 = min(PG ? min(pg.ctx[b], n_len) : n_len, n0 + per);
  const int ntiles = n1 > n0 ? (n1 - n0 + T - 1) / T : 0;
  const int nt = ntiles > wave ? (ntiles - wave + DEC_WAVES - 1) / DEC_WAVES : 0;  // this wave's
  const int8_t* kb = k + (PG ? 0 : (int64_t)bkv * n_len * D);
  constexpr int KSB = KS16 ? 2 : 4;  // K scale bytes per key
  const uint8_t* ksb = static_cast<const uint8_t*>(k_scale) + (PG ? 0 : (int64_t)bkv * n_len * KSB);
  const uint8_t* vb = static_cast<const uint8_t*>(v) + (PG ? 0 : (int64_t)bkv * n_len * C::VRB);
  __shared__ int32_t sm_bt[PG ? DEC_BT_MAX : 1];
  const int first_blk = PG ? (n0 >> pg.bs_sh) : 0;
  if constexpr (PG) {
    const int nbt = n1 > n0 ? ((n1 - 1) >> pg.bs_sh) - first_blk + 1 : 0;
    const int32_t* btb = pg.bt + (int64_t)b * pg.maxb + first_blk;
    for (int i = threadIdx.x; i < nbt; i += DEC_THREADS) sm_bt[i] = btb[i];
    __syncthreads();
  }
  // cache row of key n (clamped into the split; the repeated rows are never used)
  auto crow = [&](int n) -> int64_t {
    n = min(n, n1 - 1);
    if constexpr (PG)
      return ((int64_t)sm_bt[(n >> pg.bs_sh) - first_blk] * h_kv + kvh) * pg.bs + (n & (pg.bs - 1));
    else return n;
  };

  const int h = lane / KL, kl = lane % KL;
  const int64_t hq = (int64_t)b * h_q + (int64_t)kvh * GS + h;
  int qv[D / 4];
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    const int4 x = reinterpret_cast<const int4*>(q + hq * D)[c];
    qv[4 * c] = x.x; qv[4 * c + 1] = x.y; qv[4 * c + 2] = x.z; qv[4 * c + 3] = x.w;
  }
  const float qsc = q_scale[hq];

  // Buffer-resource copies (contiguous cache, or paged with block-aligned
  // tiles): per-lane byte offsets fixed for the kernel, the tile's first row in
  // the scalar offset; rows past the resource read as zeros, rows past the
  // split (< N) are real keys that the compute masks.
  constexpr bool BUF = !PG || PGA;
  const uint32_t res_rows = PG ? (uint32_t)pg.cache_rows : (uint32_t)n_len;
  const brsrc_t r_k = make_rsrc(kb, res_rows * D);
  const brsrc_t r_v = make_rsrc(vb, res_rows * C::VRB);
  const brsrc_t r_s = make_rsrc(ksb, res_rows * KSB);
  const brsrc_t r_vs = make_rsrc(PG ? (const void*)vsc : (const void*)ksb, PG ? res_rows * 4 : 0u);
  uint32_t kvo[C::KDMA], vvo[C::VDMA];
#pragma unroll
  for (int j = 0; j < C::KDMA; ++j) {
    const int id = j * 64 + lane, row = id / KC;
    const int c = (id % KC) ^ ((row >> KSH) & KSW);
    kvo[j] = (uint32_t)(row * D + 16 * c);
  }
#pragma unroll
  for (int j = 0; j < C::VDMA; ++j) {
    const int id = j * 64 + lane, row = id / (C::VRB / 16);
    vvo[j] = (uint32_t)(row * C::VRB + 16 * (id % (C::VRB / 16)));
  }
  // tile i of this wave = tile (wave + 4 i) of the split
  auto load_tile = [&](int i, int8_t* sb) {
    const int base = n0 + (wave + DEC_WAVES * i) * T;
    if constexpr (BUF) {
      uint32_t r0 = (uint32_t)base;  // the tile's first cache row
      if constexpr (PG) {
        const int blk = __builtin_amdgcn_readfirstlane(sm_bt[(base >> pg.bs_sh) - first_blk]);
        r0 = (uint32_t)(((int64_t)blk * h_kv + kvh) * pg.bs + (base & (pg.bs - 1)));
      }
#pragma unroll
      for (int j = 0; j < C::KDMA; ++j) buf16_to_lds(r_k, sb + j * 1024, kvo[j], r0 * D);
#pragma unroll
      for (int j = 0; j < C::VDMA; ++j)
        buf16_to_lds(r_v, sb + C::KBYTES + j * 1024, vvo[j], r0 * C::VRB);
      // lanes past the tile repeat its keys (same cache lines: no extra traffic)
      const uint32_t sl = (uint32_t)(lane % T);
      if constexpr (KS16)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r_s, (lptr_t)(sb + C::KBYTES + C::VBYTES), 2,
                                                 sl * 2, r0 * 2, 0, 0);
      else
        buf4_to_lds(r_s, sb + C::KBYTES + C::VBYTES, sl * 4, r0 * 4);
      if constexpr (PG) buf4_to_lds(r_vs, sb + C::KBYTES + C::VBYTES + 256, sl * 4, r0 * 4);
      return;
    }
#pragma unroll
    for (int j = 0; j < C::KDMA; ++j) {
      const int id = j * 64 + lane, row = id / KC;
      const int c = (id % KC) ^ ((row >> KSH) & KSW);
      __builtin_amdgcn_global_load_lds((gptr_t)(kb + crow(base + row) * D + 16 * c),
                                       (lptr_t)(sb + j * 1024), 16, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < C::VDMA; ++j) {
      const int id = j * 64 + lane, row = id / (C::VRB / 16);
      __builtin_amdgcn_global_load_lds(
          (gptr_t)(vb + crow(base + row) * C::VRB + 16 * (id % (C::VRB / 16))),
          (lptr_t)(sb + C::KBYTES + j * 1024), 16, 0, 0);
    }
    // lanes past the tile repeat its keys (same cache lines: no extra traffic)
    const int64_t sr = crow(base + (lane % T));
    if constexpr (KS16)
      __builtin_amdgcn_global_load_lds((gptr_t)(ksb + sr * 2), (lptr_t)(sb + C::KBYTES + C::VBYTES), 2, 0, 0);
    else
      __builtin_amdgcn_global_load_lds((gptr_t)(ksb + sr * 4), (lptr_t)(sb + C::KBYTES + C::VBYTES), 4, 0, 0);
    if constexpr (PG)
      __builtin_amdgcn_global_load_lds((gptr_t)(vsc + sr), (lptr_t)(sb + C::KBYTES + C::VBYTES + 256),
                                       4, 0, 0);
  };

  float m_run = -INFINITY, l_lane = 0.f, lv_lane = 0.f, oacc[CPL];  // lv: sum of p * v_scale (PG)
  float pq_sum = 0.f;  // VI8 pair path: the head's sum of the fp16 p that entered PV
#pragma unroll
  for (int e = 0; e < CPL; ++e) oacc[e] = 0.f;
  // PV4 (int8 V, D = 128, 4 query heads per KV head): the PV lanes are
  // (key-pair parity hk = lane / 32, 4 channels 4 cq .. 4 cq + 3) and each
  // covers all 4 heads, so a V byte is converted once instead of once per
  // head: per key pair 4 v_perm (fp16 denormal pairs (v + 128) * 2^-24 of the
  // two keys) and 16 v_dot2 against the heads' fp16 (p0, p1) pairs, which
  // the logit lanes stage in LDS (one 16-byte broadcast read per key pair).
  constexpr bool PV4 = SL8_DEC_PV4 && VI8 && DEC_PAIR && D == 128 && GS == 4;
  __shared__ __attribute__((aligned(16))) uint32_t pv_l[PV4 ? DEC_WAVES : 1][36];  // [8 pairs][4 heads] p2, [4] resc
  float o4[PV4 ? 4 : 1][4];  // [head][channel]
#pragma unroll
  for (int hh = 0; hh < (PV4 ? 4 : 1); ++hh)
#pragma unroll
    for (int e = 0; e < 4; ++e) o4[hh][e] = 0.f;
  const int hk = lane >> 5, cq = lane & 31;
  // v_perm selectors per channel byte e: [u(k0), 0, u(k1), 0] from (a = first
  // word read, b = second); the odd half reads key k1 first (its row lies in
  // the other 32-bank half: no bank conflict between the halves)
  uint32_t vsel[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    vsel[e] = hk == 0 ? ((uint32_t)e | (12u << 8) | ((uint32_t)(4 + e) << 16) | (12u << 24))
                      : ((uint32_t)(4 + e) | (12u << 8) | ((uint32_t)e << 16) | (12u << 24));

  auto compute_tile = [&](int i, int8_t* sb) {
    const int base = n0 + (wave + DEC_WAVES * i) * T;
    const float* kst = reinterpret_cast<const float*>(sb + C::KBYTES + C::VBYTES);
    const uint16_t* vt = reinterpret_cast<const uint16_t*>(sb + C::KBYTES);
    float s[SUB];
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < SUB; ++u) {
      const int r = u * KL + kl;
      int acc = 0;
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const int4 kr = *reinterpret_cast<const int4*>(sb + r * D + 16 * (c ^ ((r >> KSH) & KSW)));
        acc = __builtin_amdgcn_sdot4(qv[4 * c + 0], kr.x, acc, false);
        acc = __builtin_amdgcn_sdot4(qv[4 * c + 1], kr.y, acc, false);
        acc = __builtin_amdgcn_sdot4(qv[4 * c + 2], kr.z, acc, false);
        acc = __builtin_amdgcn_sdot4(qv[4 * c + 3], kr.w, acc, false);
      }
      // a 2-byte LDS DMA still fills one dword per lane (the value zero-extended)
      const float ksr = KS16 ? h2f(reinterpret_cast<const uint32_t*>(kst)[r] & 0xFFFFu) : kst[r];
      s[u] = (base + r < n1) ? ((float)acc * qsc) * ksr : -INFINITY;
      mx = fmaxf(mx, s[u]);
    }
#pragma unroll
    for (int o = 1; o < KL; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    // key `base` is valid, so mx is finite for every head
    const float mn = fmaxf(m_run, mx);
    const float resc = __builtin_amdgcn_exp2f(m_run - mn);  // first tile: exp2(-inf) = 0
    m_run = mn;
    float ps = 0.f, p[SUB];
#pragma unroll
    for (int u = 0; u < SUB; ++u) {
      p[u] = __builtin_amdgcn_exp2f(s[u] - mn);
      ps += p[u];
    }
    l_lane = l_lane * resc + ps;
    if constexpr (PG) {
      // per-token V scale: PV uses p * v_scale[key]
      const float* vst = kst + 64;
      float pvs = 0.f;
#pragma unroll
      for (int u = 0; u < SUB; ++u) {
        // keys past the sequence (p = 0) may sit in unwritten block rows whose
        // scale is not a number: select instead of multiplying
        p[u] = (base + u * KL + kl < n1) ? p[u] * vst[u * KL + kl] : 0.f;
        pvs += p[u];
      }
      lv_lane = lv_lane * resc + pvs;
    }
    if constexpr (PV4) {
      static_assert(SUB == 1 && KL == 16 && T == 16, "PV4 tile");
      typedef _Float16 v2h_t __attribute__((ext_vector_type(2)));
      // this lane's p (fp16, as it enters PV) into the wave's LDS slot: pair
      // kl / 2, head h, key kl & 1; the head's rescale factor after the pairs
      const _Float16 ph = (_Float16)p[0];
      pq_sum = pq_sum * resc + (float)ph;
      uint16_t* pt = reinterpret_cast<uint16_t*>(&pv_l[wave][0]);
      pt[(kl >> 1) * 8 + 2 * h + (kl & 1)] = __builtin_bit_cast(uint16_t, ph);
      if (kl == 0) reinterpret_cast<float*>(&pv_l[wave][32])[h] = resc;
      // (this wave's own LDS writes: read back in order)
      const float4 rs = *reinterpret_cast<const float4*>(&pv_l[wave][32]);
      const float rsh[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
      for (int hh = 0; hh < 4; ++hh)
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[hh][e] *= rsh[hh];
      const uint8_t* vbt = reinterpret_cast<const uint8_t*>(vt);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int pp = 2 * j + hk;  // key pair 2 pp, 2 pp + 1
        const uint4 pv = *reinterpret_cast<const uint4*>(&pv_l[wave][4 * pp]);
        const uint32_t pw[4] = {pv.x, pv.y, pv.z, pv.w};
        const uint32_t wa = *reinterpret_cast<const uint32_t*>(vbt + (2 * pp + hk) * D + 4 * cq) ^ 0x80808080u;
        const uint32_t wb = *reinterpret_cast<const uint32_t*>(vbt + (2 * pp + 1 - hk) * D + 4 * cq) ^ 0x80808080u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t pr = __builtin_amdgcn_perm(wb, wa, vsel[e]);
#pragma unroll
          for (int hh = 0; hh < 4; ++hh)
            o4[hh][e] = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h_t, pw[hh]), __builtin_bit_cast(v2h_t, pr),
                                               o4[hh][e], false);
        }
      }
      return;
    }
#pragma unroll
    for (int e = 0; e < CPL; ++e) oacc[e] *= resc;
    if constexpr (VI8 && DEC_PAIR) {
      // Two keys per step: one v_perm per channel packs the unsigned codes
      // u = v + 128 of keys k0, k1 as the fp16 pair (u0, u1) * 2^-24 (exact
      // fp16 denormals, byte over a zero byte), and v_dot2_f32_f16 against
      // the fp16 pair (p0, p1) accumulates both keys. The 2^24 factor and the
      // 128 * sum(p) offset are removed once per split.
      pq_sum *= resc;
      typedef _Float16 v2h_t __attribute__((ext_vector_type(2)));
      const v2h_t one2 = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
      for (int u = 0; u < SUB; ++u) {
        static_for<0, KL / 2>([&](auto rc) {
          constexpr int rr = 2 * decltype(rc)::value;
          const float pk0 = lane_bcast<KL, rr>(p[u]);
          const float pk1 = lane_bcast<KL, rr + 1>(p[u]);
          const v2h_t pp = {(_Float16)pk0, (_Float16)pk1};
          pq_sum = __builtin_amdgcn_fdot2(pp, one2, pq_sum, false);
          const uint8_t* r0 = reinterpret_cast<const uint8_t*>(vt) + (u * KL + rr) * D + kl * CPL;
          const uint8_t* r1 = r0 + D;
          uint32_t w0[CPL / 4], w1[CPL / 4];
          if constexpr (CPL % 16 == 0) {
#pragma unroll
            for (int c16 = 0; c16 < CPL; c16 += 16) {
              const uint4 x0 = *reinterpret_cast<const uint4*>(r0 + c16);
              const uint4 x1 = *reinterpret_cast<const uint4*>(r1 + c16);
              w0[c16 / 4] = x0.x; w0[c16 / 4 + 1] = x0.y; w0[c16 / 4 + 2] = x0.z; w0[c16 / 4 + 3] = x0.w;
              w1[c16 / 4] = x1.x; w1[c16 / 4 + 1] = x1.y; w1[c16 / 4 + 2] = x1.z; w1[c16 / 4 + 3] = x1.w;
            }
          } else if constexpr (CPL == 8) {
            const uint2 x0 = *reinterpret_cast<const uint2*>(r0);
            const uint2 x1 = *reinterpret_cast<const uint2*>(r1);
            w0[0] = x0.x; w0[1] = x0.y;
            w1[0] = x1.x; w1[1] = x1.y;
          } else {
            w0[0] = *reinterpret_cast<const uint32_t*>(r0);
            w1[0] = *reinterpret_cast<const uint32_t*>(r1);
          }
#pragma unroll
          for (int c = 0; c < CPL / 4; ++c) {
            const uint32_t a = w0[c] ^ 0x80808080u, bq = w1[c] ^ 0x80808080u;
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
              // bytes: [a_bb, 0, b_bb, 0] (selector 12 = zero byte; 0-3 = a, 4-7 = bq)
              const uint32_t sel = (uint32_t)bb | (12u << 8) | ((uint32_t)(4 + bb) << 16) | (12u << 24);
              const uint32_t pr = __builtin_amdgcn_perm(bq, a, sel);
              oacc[4 * c + bb] = __builtin_amdgcn_fdot2(pp, __builtin_bit_cast(v2h_t, pr), oacc[4 * c + bb], false);
            }
          }
        });
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < SUB; ++u) {
      static_for<0, KL>([&](auto rc) {
        constexpr int rr = decltype(rc)::value;
        // P of key u*KL+rr (held by lane h*KL+rr) to every lane of head h
        const float pk = lane_bcast<KL, rr>(p[u]);
        if constexpr (VI8) {
          // int8 codes v -> fp16 1024 + (v + 128), exact: flip the sign bit
          // (u = v + 128 as an unsigned byte) and pair it with the exponent
          // byte 0x64 (fp16 0x64uu = 1024 + uu); the 1152 * sum(p) offset is
          // removed once at the end
          const uint8_t* vrow8 = reinterpret_cast<const uint8_t*>(vt) + (u * KL + rr) * D + kl * CPL;
          uint32_t vw[CPL / 4];
          if constexpr (CPL % 16 == 0) {
#pragma unroll
            for (int c16 = 0; c16 < CPL; c16 += 16) {
              const uint4 x = *reinterpret_cast<const uint4*>(vrow8 + c16);
              vw[c16 / 4] = x.x; vw[c16 / 4 + 1] = x.y; vw[c16 / 4 + 2] = x.z; vw[c16 / 4 + 3] = x.w;
            }
          } else if constexpr (CPL == 8) {
            const uint2 x = *reinterpret_cast<const uint2*>(vrow8);
            vw[0] = x.x; vw[1] = x.y;
          } else {
            vw[0] = *reinterpret_cast<const uint32_t*>(vrow8);
          }
#pragma unroll
          for (int c = 0; c < CPL / 4; ++c) {
            const uint32_t w = vw[c] ^ 0x80808080u;
            const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
            const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
            oacc[4 * c] = fmaf(pk, h2f(lo & 0xFFFF), oacc[4 * c]);
            oacc[4 * c + 1] = fmaf(pk, h2f(lo >> 16), oacc[4 * c + 1]);
            oacc[4 * c + 2] = fmaf(pk, h2f(hi & 0xFFFF), oacc[4 * c + 2]);
            oacc[4 * c + 3] = fmaf(pk, h2f(hi >> 16), oacc[4 * c + 3]);
          }
          return;
        }
        const uint16_t* vrow = vt + (u * KL + rr) * D + kl * CPL;
        uint32_t vw[CPL / 2];
        if constexpr (CPL % 8 == 0) {
#pragma unroll
          for (int c8 = 0; c8 < CPL; c8 += 8) {
            const uint4 x = *reinterpret_cast<const uint4*>(vrow + c8);
            vw[c8 / 2] = x.x; vw[c8 / 2 + 1] = x.y; vw[c8 / 2 + 2] = x.z; vw[c8 / 2 + 3] = x.w;
          }
        } else {
          const uint2 x = *reinterpret_cast<const uint2*>(vrow);
          vw[0] = x.x; vw[1] = x.y;
        }
#pragma unroll
        for (int c = 0; c < CPL / 2; ++c) {
          oacc[2 * c] = fmaf(pk, h2f(vw[c] & 0xFFFF), oacc[2 * c]);
          oacc[2 * c + 1] = fmaf(pk, h2f(vw[c] >> 16), oacc[2 * c + 1]);
        }
      });
    }
  };

  // Copies per tile per lane: KDMA + VDMA + 1 (+1 paged), all from this wave. Before
  // tile i is read, wait until only the copies of tiles i+1 .. i+NB-2 (issued
  // later) may still be in flight; vmcnt retires in issue order.
  constexpr int AHEAD = (NB - 1) * (C::KDMA + C::VDMA + (PG ? 2 : 1));
  static_assert(AHEAD < 64, "vmcnt range");
  constexpr unsigned WAIT_AHEAD = 0x0F70u | (AHEAD & 15) | ((AHEAD >> 4) << 14);
  // The Q loads above were issued before any copy, so the in-order vmcnt waits
  // below also cover them.
#pragma unroll
  for (int i = 0; i < NB - 1; ++i)
    if (i < nt) load_tile(i, stage(i));
  for (int i0 = 0; i0 < nt; i0 += NB) {
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int i = i0 + u;
      if (i < nt) {
        if (i + NB - 1 < nt) {
          // refills the stage read by tile i-1 (already consumed by this wave)
          load_tile(i + NB - 1, stage((u + NB - 1) % NB));
          __builtin_amdgcn_s_waitcnt(WAIT_AHEAD);
        } else {
          __builtin_amdgcn_s_waitcnt(0x0F70);
        }
        compute_tile(i, stage(u));
      }
    }
  }

  // ---- per-wave state -> LDS (this wave's own stage-0 area), then LSE merge ----
#pragma unroll
  for (int o = 1; o < KL; o <<= 1) l_lane += __shfl_xor(l_lane, o, 64);
  if constexpr (PV4) {
    // the two key-parity halves, then per head: codes entered PV as
    // (v + 128) * 2^-24 against the fp16 p (pq_sum: their sum per head)
#pragma unroll
    for (int o = 1; o < KL; o <<= 1) pq_sum += __shfl_xor(pq_sum, o, 64);
    float pqh[4];
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) pqh[hh] = __shfl(pq_sum, hh * KL, 64);
#pragma unroll
    for (int hh = 0; hh < 4; ++hh)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = o4[hh][e] + __shfl_xor(o4[hh][e], 32, 64);
        v = v * 16777216.f - 128.f * pqh[hh];
        if constexpr (!PG) v *= vsc[(int64_t)bkv * D + 4 * cq + e];
        o4[hh][e] = v;
      }
  } else if constexpr (VI8 && DEC_PAIR) {
    // codes entered PV as (v + 128) * 2^-24 against the fp16 p: rescale and
    // remove the 128 offset weighted by exactly those p
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      oacc[e] = oacc[e] * 16777216.f - 128.f * pq_sum;
      if constexpr (!PG) oacc[e] *= vsc[(int64_t)bkv * D + kl * CPL + e];
    }
  } else if constexpr (PG) {
    // remove the 1152 offset per key, weighted like the p that entered PV
#pragma unroll
    for (int o = 1; o < KL; o <<= 1) lv_lane += __shfl_xor(lv_lane, o, 64);
#pragma unroll
    for (int e = 0; e < CPL; ++e) oacc[e] -= 1152.f * lv_lane;
  } else if constexpr (VI8) {
    // remove the 1152 offset per key (l_lane is now the head's sum of p,
    // rescaled exactly like oacc) and fold in the per-channel scale
#pragma unroll
    for (int e = 0; e < CPL; ++e)
      oacc[e] = (oacc[e] - 1152.f * l_lane) * vsc[(int64_t)bkv * D + kl * CPL + e];
  }
  float* red = reinterpret_cast<float*>(st0);  // [wave][GS][D] o, then [wave][GS] m, l
  float* ro = red + wave * GS * D;
  float* rm = red + DEC_WAVES * GS * D + wave * GS;
  float* rl = red + DEC_WAVES * GS * D + DEC_WAVES * GS + wave * GS;
  __syncthreads();  // every wave is past its last read of stage 0
  if constexpr (PV4) {
    if (hk == 0) {
#pragma unroll
      for (int hh = 0; hh < 4; ++hh)
        *reinterpret_cast<float4*>(ro + hh * D + 4 * cq) = make_float4(o4[hh][0], o4[hh][1], o4[hh][2], o4[hh][3]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < CPL; e += 4)
      *reinterpret_cast<float4*>(ro + h * D + kl * CPL + e) =
          make_float4(oacc[e], oacc[e + 1], oacc[e + 2], oacc[e + 3]);
  }
  if (kl == 0) {
    rm[h] = m_run;
    rl[h] = l_lane;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < GS * D; idx += DEC_THREADS) {
    const int hh = idx / D, d = idx % D;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < DEC_WAVES; ++w) mm = fmaxf(mm, red[DEC_WAVES * GS * D + w * GS + hh]);
    float acc = 0.f, den = 0.f;
    if (mm != -INFINITY) {
#pragma unroll
      for (int w = 0; w < DEC_WAVES; ++w) {
        const float mw = red[DEC_WAVES * GS * D + w * GS + hh];
        const float wt = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - mm);
        acc += red[w * GS * D + hh * D + d] * wt;
        den += red[DEC_WAVES * GS * D + DEC_WAVES * GS + w * GS + hh] * wt;
      }
    }
    const int64_t row = (int64_t)split * bhq + (int64_t)b * h_q + (int64_t)kvh * GS + hh;
    o_part[row * D + d] = acc;
    if (d == 0) {
      m_part[row] = mm == -INFINITY ? DEC_NEG_INF : mm;
      l_part[row] = den;
    }
  }
}

template <int D, int G, bool VI8, bool PG, bool KS16>
void launch_split(dim3 grid, const int8_t* q, const float* qs, const int8_t* k, const void* ks,
                  const void* v, const float* vsc, float* op, float* mp, float* lp, int N, int ns,
                  int hq, int hkv, int gsz, int bhq, const PagedArgs& pg, hipStream_t st) {
  decode_split_kernel<D, G, VI8, PG, KS16><<<grid, DEC_THREADS, 0, st>>>(
      q, qs, k, ks, v, vsc, op, mp, lp, N, ns, hq, hkv, gsz, bhq, pg);
}

template <int D, bool VI8, bool PG = false, bool KS16 = false>
void launch_d(int G, dim3 grid, const int8_t* q, const float* qs, const int8_t* k,
              const void* ks, const void* v, const float* vsc, float* op, float* mp, float* lp,
              int N, int ns, int hq, int hkv, int gsz, int bhq, hipStream_t st,
              const PagedArgs& pg = PagedArgs{nullptr, nullptr, 0, 1, 0, 0}) {
#define SL8_SPLIT(GG) \
  launch_split<D, GG, VI8, PG, KS16>(grid, q, qs, k, ks, v, vsc, op, mp, lp, N, ns, hq, hkv, gsz, bhq, pg, st)
  switch (G) {
    case 1: SL8_SPLIT(1); break;
    case 2: SL8_SPLIT(2); break;
    case 4: SL8_SPLIT(4); break;
    default: SL8_SPLIT(8); break;
  }
#undef SL8_SPLIT
}

int group_width(int gsz) { return gsz >= 8 ? 8 : gsz >= 4 ? 4 : gsz >= 2 ? 2 : 1; }

}  // namespace
}  // namespace sl8

using namespace sl8;

// Auto split count: enough workgroups to cover 256 CUs ~8 times, at least 256
// keys (one 64-key tile per wave) per split, at most DEC_MAX_SPLITS.
extern "C" int sl8_choose_num_splits(int64_t N, int64_t B, int64_t Hkv) {
  if (N <= 0 || B <= 0 || Hkv <= 0) return 1;
  const int64_t groups = B * Hkv;
  int64_t s = (2048 + groups - 1) / groups;
  const int64_t s_hi = (N + 255) / 256;
  if (s > s_hi) s = s_hi;
  if (s < 1) s = 1;
  if (s > DEC_MAX_SPLITS) s = DEC_MAX_SPLITS;
  return (int)s;
}

extern "C" size_t sl8_attn_int8_decode_workspace(int64_t B, int64_t Hq, int64_t D,
                                                 int64_t num_splits) {
  if (B <= 0 || Hq <= 0 || D <= 0 || num_splits <= 0) return 0;
  return (size_t)(num_splits * B * Hq * (D + 2)) * sizeof(float);
}

namespace sl8 {
namespace {

// Split kernels + combine. v: fp16 [B,Hkv,N,D], or int8 with vsc [B,Hkv,D] (VI8).
// k_scale: fp32 per key, or fp16 with KS16.
template <bool VI8, bool KS16 = false>
int decode_launch(const int8_t* q, const float* q_scale, const int8_t* k, const void* k_scale,
                  const void* v, const float* vsc, void* out, int64_t B, int64_t Hq, int64_t Hkv,
                  int64_t N, int64_t D, int64_t num_splits, void* workspace, hipStream_t st) {
  // one KV head's cache is addressed by 32-bit buffer offsets in the streaming kernel
  SL8_CHECK_ARG(N * D * (VI8 ? 1 : 2) < (1LL << 31), "fni8 decode: shape too large (N=%lld)",
                (long long)N);
  const int ns = (int)num_splits, bhq = (int)(B * Hq), gsz = (int)(Hq / Hkv);
  const int G = group_width(gsz);
  float* op = static_cast<float*>(workspace);
  float* mp = op + (size_t)ns * bhq * D;
  float* lp = mp + (size_t)ns * bhq;
  const dim3 grid((unsigned)ns, (unsigned)(B * Hkv), (unsigned)((gsz + G - 1) / G));
  // D = 32 (too few channels for the streaming kernel's lane maps) takes the
  // per-key split kernel
  if (D != 32 && ((gsz == 2 && D == 128) || gsz == 4 || gsz == 8)) {
    const dim3 g2((unsigned)ns, (unsigned)(B * Hkv));
#define SL8_WAVE(DD, GS, NB)                                                                     \
    decode_wave_kernel<DD, GS, NB, VI8, false, KS16><<<g2, DEC_THREADS, 0, st>>>(                    \
        q, q_scale, k, k_scale, v, vsc, op, mp, lp, (int)N, ns, (int)Hq, (int)Hkv, bhq,       \
        PagedArgs{nullptr, nullptr, 0, 1, 0, 0})
#define SL8_WAVE_D(GS)                         \
    if (D == 64) SL8_WAVE(64, GS, 4);          \
    else if (D == 128) SL8_WAVE(128, GS, 3);   \
    else SL8_WAVE(256, GS, 3);
    switch (gsz) {
      case 2: SL8_WAVE(128, 2, 3); break;
      case 4: SL8_WAVE_D(4); break;
      default: SL8_WAVE_D(8); break;
    }
#undef SL8_WAVE_D
#undef SL8_WAVE
  } else switch (D) {
    case 32: launch_d<32, VI8, false, KS16>(G, grid, q, q_scale, k, k_scale, v, vsc, op, mp, lp, (int)N, ns, (int)Hq, (int)Hkv, gsz, bhq, st); break;
    case 64: launch_d<64, VI8, false, KS16>(G, grid, q, q_scale, k, k_scale, v, vsc, op, mp, lp, (int)N, ns, (int)Hq, (int)Hkv, gsz, bhq, st); break;
    case 128: launch_d<128, VI8, false, KS16>(G, grid, q, q_scale, k, k_scale, v, vsc, op, mp, lp, (int)N, ns, (int)Hq, (int)Hkv, gsz, bhq, st); break;
    default: launch_d<256, VI8, false, KS16>(G, grid, q, q_scale, k, k_scale, v, vsc, op, mp, lp, (int)N, ns, (int)Hq, (int)Hkv, gsz, bhq, st); break;
  }
  SL8_CHECK_LAUNCH("attn_int8_decode split");
  launch_combine((int)D, bhq, st, op, mp, lp, static_cast<uint16_t*>(out), ns, bhq);
  SL8_CHECK_LAUNCH("attn_int8_decode combine");
  return SL8_OK;
}

}  // namespace
}  // namespace sl8

extern "C" int sl8_attn_int8_decode(const int8_t* q, const float* q_scale, const int8_t* k,
                                    const float* k_scale, const void* v, void* out, int64_t B,
                                    int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                                    int64_t num_splits, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  clear_error();
  SL8_CHECK_ARG(B >= 0 && Hq >= 0 && Hkv > 0 && N >= 0, "fni8 decode: bad shape");
  SL8_CHECK_ARG(Hq % Hkv == 0, "fni8 decode: H_q must be divisible by H_kv (GQA)");
  SL8_CHECK_ARG(D == 32 || D == 64 || D == 128 || D == 256, "fni8 decode: head dim must be 32/64/128/256, got %lld",
                (long long)D);
  if (num_splits < 0) num_splits = sl8_choose_num_splits(N, B, Hkv);
  SL8_CHECK_ARG(num_splits >= 1 && num_splits <= DEC_MAX_SPLITS,
                "fni8 decode: num_splits must be 1..%d, got %lld", DEC_MAX_SPLITS,
                (long long)num_splits);
  SL8_CHECK_ARG(B * Hq < (1LL << 31) && N < (1LL << 31), "fni8 decode: shape too large");
  if (B == 0 || Hq == 0) return SL8_OK;
  SL8_CHECK_ARG(N > 0, "fni8 decode: empty KV cache (the caller zero-fills the output)");
  SL8_CHECK_ARG(q && q_scale && k && k_scale && v && out, "fni8 decode: null pointer");
  SL8_CHECK_ARG(aligned(q, 16) && aligned(k, 16) && aligned(v, 16),
                "fni8 decode: q/k/v must be 16-byte aligned");
  const size_t need = sl8_attn_int8_decode_workspace(B, Hq, D, num_splits);
  SL8_CHECK_ARG(workspace && workspace_bytes >= need && aligned(workspace, 16),
                "fni8 decode: workspace needs %zu bytes", need);
  return decode_launch<false>(q, q_scale, k, k_scale, v, nullptr, out, B, Hq, Hkv, N, D,
                              num_splits, workspace, static_cast<hipStream_t>(stream));
}

// fp16 per-token K scales (BASELINE config 3's cache format: half the scale
// bytes of the reference's fp32 contract, attn_decode.cu:174-175). Otherwise
// identical to sl8_attn_int8_decode: the scale is widened to fp32 exactly
// before the same arithmetic.
extern "C" int sl8_attn_int8_decode_ks16(const int8_t* q, const float* q_scale, const int8_t* k,
                                         const void* k_scale_f16, const void* v, void* out,
                                         int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                                         int64_t num_splits, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  clear_error();
  SL8_CHECK_ARG(B >= 0 && Hq >= 0 && Hkv > 0 && N >= 0, "fni8 decode: bad shape");
  SL8_CHECK_ARG(Hq % Hkv == 0, "fni8 decode: H_q must be divisible by H_kv (GQA)");
  SL8_CHECK_ARG(D == 32 || D == 64 || D == 128 || D == 256,
                "fni8 decode: head dim must be 32/64/128/256, got %lld", (long long)D);
  if (num_splits < 0) num_splits = sl8_choose_num_splits(N, B, Hkv);
  SL8_CHECK_ARG(num_splits >= 1 && num_splits <= DEC_MAX_SPLITS,
                "fni8 decode: num_splits must be 1..%d, got %lld", DEC_MAX_SPLITS,
                (long long)num_splits);
  SL8_CHECK_ARG(B * Hq < (1LL << 31) && N < (1LL << 31), "fni8 decode: shape too large");
  if (B == 0 || Hq == 0) return SL8_OK;
  SL8_CHECK_ARG(N > 0, "fni8 decode: empty KV cache (the caller zero-fills the output)");
  SL8_CHECK_ARG(q && q_scale && k && k_scale_f16 && v && out, "fni8 decode: null pointer");
  SL8_CHECK_ARG(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(k_scale_f16, 2),
                "fni8 decode: q/k/v must be 16-byte aligned");
  const size_t need = sl8_attn_int8_decode_workspace(B, Hq, D, num_splits);
  SL8_CHECK_ARG(workspace && workspace_bytes >= need && aligned(workspace, 16),
                "fni8 decode: workspace needs %zu bytes", need);
  return decode_launch<false, true>(q, q_scale, k, k_scale_f16, v, nullptr, out, B, Hq, Hkv, N, D,
                                    num_splits, workspace, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// Allocation-free split-KV decode: the per-split partials (O, m, l) live in a
// file-scope device array instead of a caller workspace, for callers that may
// not allocate device memory (HIP graph capture, serving loops). Each device
// holds its own copy of the array; its address is looked up once per device
// with hipGetSymbolAddress (the array's name is a host-side stand-in, never a
// device address) and kept in noalloc_scratch_ptr[]. Every call on a device
// shares that device's array: calls that overlap on one device (different
// streams, or other host threads) race on it. The decode kernels write every
// partial they merge (empty splits write the m = -1e30 sentinel), so nothing
// has to start at zero.
// ---------------------------------------------------------------------------
namespace sl8 {
namespace {
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)8 << 20;
constexpr int NOALLOC_MAX_DEVICES = 64;
__device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];
void* noalloc_scratch_ptr[NOALLOC_MAX_DEVICES];
std::mutex noalloc_mu;

int noalloc_scratch(void** out) {
  int dev = -1;
  const hipError_t e0 = hipGetDevice(&dev);
  SL8_CHECK_ARG(e0 == hipSuccess, "fni8 decode_noalloc: hipGetDevice failed: %s", hipGetErrorString(e0));
  SL8_CHECK_ARG(dev >= 0 && dev < NOALLOC_MAX_DEVICES, "fni8 decode_noalloc: device %d out of range",
                dev);
  std::lock_guard<std::mutex> lock(noalloc_mu);
  if (!noalloc_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e1 = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    SL8_CHECK_ARG(e1 == hipSuccess, "fni8 decode_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                  hipGetErrorString(e1));
    SL8_CHECK_ARG(p != nullptr, "fni8 decode_noalloc: no device address for the scratch array");
    noalloc_scratch_ptr[dev] = p;
  }
  *out = noalloc_scratch_ptr[dev];
  return SL8_OK;
}
}  // namespace
}  // namespace sl8

extern "C" size_t sl8_attn_int8_decode_noalloc_max_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

extern "C" int sl8_attn_int8_decode_noalloc(const int8_t* q, const float* q_scale, const int8_t* k,
                                            const float* k_scale, const void* v, void* out,
                                            int64_t B, int64_t Hq, int64_t Hkv, int64_t N,
                                            int64_t D, int64_t num_splits, void* stream) {
  clear_error();
  // same checks and split choice as sl8_attn_int8_decode; the partials must
  // fit the scratch array
  SL8_CHECK_ARG(B >= 0 && Hq >= 0 && Hkv > 0 && N >= 0, "fni8 decode: bad shape");
  SL8_CHECK_ARG(D == 32 || D == 64 || D == 128 || D == 256, "fni8 decode: head dim must be 32/64/128/256, got %lld",
                (long long)D);
  int64_t ns = num_splits < 0 ? (Hkv > 0 ? sl8_choose_num_splits(N, B, Hkv) : 1) : num_splits;
  SL8_CHECK_ARG(ns >= 1 && ns <= DEC_MAX_SPLITS, "fni8 decode: num_splits must be 1..%d, got %lld",
                DEC_MAX_SPLITS, (long long)ns);
  const size_t need = sl8_attn_int8_decode_workspace(B, Hq, D, ns);
  SL8_CHECK_ARG(need <= NOALLOC_SCRATCH_BYTES,
                "fni8 decode_noalloc: partials need %zu bytes, above the %zu-byte scratch array "
                "(fewer splits or a smaller batch; or sl8_attn_int8_decode with a workspace)",
                need, NOALLOC_SCRATCH_BYTES);
  if (B == 0 || Hq == 0) return SL8_OK;
  void* ws = nullptr;
  const int rc = noalloc_scratch(&ws);
  if (rc) return rc;
  return sl8_attn_int8_decode(q, q_scale, k, k_scale, v, out, B, Hq, Hkv, N, D, ns, ws,
                              NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int sl8_attn_int8_decode_kv8(const int8_t* q, const float* q_scale, const int8_t* k,
                                        const float* k_scale, const int8_t* v, const float* v_scale,
                                        void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t N,
                                        int64_t D, int64_t num_splits, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  clear_error();
  SL8_CHECK_ARG(B >= 0 && Hq >= 0 && Hkv > 0 && N >= 0, "fni8 decode_kv8: bad shape");
  SL8_CHECK_ARG(Hq % Hkv == 0, "fni8 decode_kv8: H_q must be divisible by H_kv (GQA)");
  SL8_CHECK_ARG(D == 32 || D == 64 || D == 128 || D == 256, "fni8 decode_kv8: head dim must be 32/64/128/256, got %lld",
                (long long)D);
  if (num_splits < 0) num_splits = sl8_choose_num_splits(N, B, Hkv);
  SL8_CHECK_ARG(num_splits >= 1 && num_splits <= DEC_MAX_SPLITS,
                "fni8 decode_kv8: num_splits must be 1..%d, got %lld", DEC_MAX_SPLITS,
                (long long)num_splits);
  SL8_CHECK_ARG(B * Hq < (1LL << 31) && N < (1LL << 31), "fni8 decode_kv8: shape too large");
  if (B == 0 || Hq == 0) return SL8_OK;
  SL8_CHECK_ARG(N > 0, "fni8 decode_kv8: empty KV cache (the caller zero-fills the output)");
  SL8_CHECK_ARG(q && q_scale && k && k_scale && v && v_scale && out, "fni8 decode_kv8: null pointer");
  SL8_CHECK_ARG(aligned(q, 16) && aligned(k, 16) && aligned(v, 16),
                "fni8 decode_kv8: q/k/v must be 16-byte aligned");
  const size_t need = sl8_attn_int8_decode_workspace(B, Hq, D, num_splits);
  SL8_CHECK_ARG(workspace && workspace_bytes >= need && aligned(workspace, 16),
                "fni8 decode_kv8: workspace needs %zu bytes", need);
  return decode_launch<true>(q, q_scale, k, k_scale, v, v_scale, out, B, Hq, Hkv, N, D,
                             num_splits, workspace, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// Paged KV cache (reference csrc/include/attn_paged_decode.cuh,
// csrc/kernel/attn_paged_decode.cu)
// ---------------------------------------------------------------------------
namespace sl8 {
namespace {

// Quantize-on-write: one wave per (batch, KV head) row of the new token.
// scale = amax / 127 (IEEE division), 1 for a zero row; code = rint(clamp(x /
// scale, +-127)); stored at flat slot = block * bs + offset.
template <int D>
__global__ void __launch_bounds__(64)
kv_write_paged_kernel(const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
                      const int32_t* __restrict__ slot_mapping, int8_t* __restrict__ k_cache,
                      float* __restrict__ k_scale, int8_t* __restrict__ v_cache,
                      float* __restrict__ v_scale, int h_kv, int bs) {
  constexpr int E = D >= 64 ? D / 64 : 1;  // elements per lane
  const int lane = threadIdx.x;
  const bool act = lane * E < D;  // D = 32: lanes 32..63 idle
  const int64_t bh = blockIdx.x;
  const int64_t b = bh / h_kv, h = bh % h_kv;
  float kx[E], vx[E];
  float ka = 0.f, va = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    kx[e] = act ? h2f(k_new[bh * D + lane * E + e]) : 0.f;
    vx[e] = act ? h2f(v_new[bh * D + lane * E + e]) : 0.f;
    ka = fmaxf(ka, fabsf(kx[e]));
    va = fmaxf(va, fabsf(vx[e]));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    ka = fmaxf(ka, __shfl_xor(ka, o, 64));
    va = fmaxf(va, __shfl_xor(va, o, 64));
  }
  const float ks = ka > 0.f ? __fdiv_rn(ka, 127.f) : 1.f;
  const float vs = va > 0.f ? __fdiv_rn(va, 127.f) : 1.f;
  const int64_t slot = slot_mapping[b];
  const int64_t row = ((slot / bs) * h_kv + h) * bs + slot % bs;
#pragma unroll
  for (int e = 0; e < E && act; ++e) {
    k_cache[row * D + lane * E + e] = (int8_t)rintf(fminf(fmaxf(__fdiv_rn(kx[e], ks), -127.f), 127.f));
    v_cache[row * D + lane * E + e] = (int8_t)rintf(fminf(fmaxf(__fdiv_rn(vx[e], vs), -127.f), 127.f));
  }
  if (lane == 0) {
    k_scale[row] = ks;
    v_scale[row] = vs;
  }
}

// ---------------------------------------------------------------------------
// K8V3 paged decode (reference attn_paged_decode.cuh:114-257 with LowbitV,
// attn_paged_decode.cu:229-330). K and the split / softmax / merge contract are
// those of the paged int8 decode; V is a 3-bit Lloyd-Max store per token:
// v_packed [rows, 3D/32] u32 holds the code of channel d at bits 3d..3d+2 of
// the row's LSB-first bit stream, v_norm [rows, D/128] fp32 one L2 norm per
// 128-channel block, codebook [8] fp32; channel d of token row r is
//   v = fp16_rn(fp32(codebook[code] * v_norm[r][d / 128])).
//
// One wave streams 64-key tiles of its split. Lane roles: (g4, col) =
// (lane / 16, lane % 16) for the MFMAs, key = lane for the per-key work,
// (kr, kh) = (lane % 32, lane / 32) for the V dequantisation.
//   * QK: S^T (64 keys x 16 head columns) on v_mfma_i32_16x16x64_i8 straight
//     from the loads: the A operand of key block kb is key 16 kb + col,
//     bytes 16 g4 .. +15 of each 64-byte K slice, which is also a coalesced
//     load (64 contiguous bytes per row and instruction); Q^T (B) stays in
//     registers, head columns >= G zero;
//   * softmax in the MFMA output layout: lane (g4, col) holds keys
//     16 kb + 4 g4 + i of head col; logit = (acc * k_scale) * q_scale, the
//     tile max over the lane's 16 values and the 4 lanes of the column; p
//     stored as fp16 in LDS, one 64-key row per head (rows G..15 stay zero);
//   * value tables (key = lane): fp16 of codebook[i] * norm for i = 0..7 per
//     128-channel block, as a low-byte plane (2 dwords) and a high-byte plane
//     (2 dwords), handed to the dequantising lanes by v_permlane32_swap;
//   * PV in two 32-key halves: lane (kr, kh) loads the code bits of channel
//     half kh of key 32 h + kr, turns 8 codes at a time into byte selectors
//     0..7, picks the fp16 values out of the table planes with v_perm_b32, and
//     writes the half row to an 8 KB (D = 128) LDS tile, read back transposed
//     (ds_read_b64_tr_b16) as the A operand of v_mfma_f32_16x16x32_f16
//     (16 channels x 32 keys) against P^T (32 keys x 16 heads).
// Each of the next tile's loads goes into the registers of the current tile's
// input right after its last use, so they are in flight during the rest of
// the tile. P enters the MFMA as fp16 (relative rounding 2^-11 per
// probability; the reference multiplies the fp32 p); the V values are exactly
// the reference's.
template <int D, int G>
struct K3Smem {
  static constexpr int PP = 72;  // P row pitch in halves (64 keys + 8: bank spread)
  int q[G][D / 4];
  float qs[G];
  // 16-byte aligned: 16-byte tile writes and the transposed 8-byte reads need
  // naturally aligned LDS addresses (q and qs end at 4 mod 16 when G = 1)
  union alignas(16) {
    struct {
      uint16_t v[DEC_WAVES][32 * D];   // fp16 V half tile [32 keys][D], 32-byte chunks swizzled
      uint16_t p[DEC_WAVES][16 * PP];  // fp16 P [16 heads][64 keys]
      float ks[DEC_WAVES][DEC_TILE];   // the tile's k_scale
    } t;
    struct {
      float m[DEC_WAVES][G];
      float l[DEC_WAVES][G];
      float o[DEC_WAVES][G][D];
    } r;
  };
};

// four 3-bit fields (bits 0..11) -> the low 3 bits of four bytes
__device__ __forceinline__ uint32_t spread3x4(uint32_t a) {
  const uint32_t t = (a & 0x3fu) | ((a & 0xfc0u) << 10);
  return (t & 0x00070007u) | ((t & 0x00380038u) << 5);
}

// 8 fp16 values (channel order) of the 8 codes in bits 0..23 of x, looked up
// in the table planes tb = {lo 0-3, lo 4-7, hi 0-3, hi 4-7}
__device__ __forceinline__ uint4 lm3_lookup8(uint32_t x, const uint4& tb) {
  uint4 r;
  const uint32_t s0 = spread3x4(x & 0xfffu), s1 = spread3x4((x >> 12) & 0xfffu);
  uint32_t lo = __builtin_amdgcn_perm(tb.y, tb.x, s0);
  uint32_t hi = __builtin_amdgcn_perm(tb.w, tb.z, s0);
  r.x = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
  r.y = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
  lo = __builtin_amdgcn_perm(tb.y, tb.x, s1);
  hi = __builtin_amdgcn_perm(tb.w, tb.z, s1);
  r.z = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
  r.w = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
  return r;
}

__device__ __forceinline__ uint32_t swap32_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_permlane32_swap(a, b, false, false)[0];
}
__device__ __forceinline__ uint32_t swap32_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_permlane32_swap(a, b, false, false)[1];
}

template <int D, int G>
// workgroups per CU: the most that fit without spills
__global__ void __launch_bounds__(DEC_THREADS, (D == 128 && G <= 4) ? 3 : 2)
k8v3_split_kernel(const int8_t* __restrict__ q, const float* __restrict__ q_scale,
                  const int8_t* __restrict__ k, const float* __restrict__ k_scale,
                  const uint32_t* __restrict__ vpk, const float* __restrict__ vnorm,
                  const float* __restrict__ codebook, float* __restrict__ o_part,
                  float* __restrict__ m_part, float* __restrict__ l_part, int n_len,
                  int n_splits, int h_q, int h_kv, int gsz, int bhq, const PagedArgs pg) {
  static_assert(G <= 16, "S^T and P^T have 16 head columns");
  using SM = K3Smem<D, G>;
  constexpr int D4 = D / 4;
  constexpr int KS = D / 64;      // 64-channel QK steps
  constexpr int VW = 3 * D / 32;  // code dwords per row
  constexpr int VB = D / 128;     // norms per row
  constexpr int HW = VW / 2;      // code dwords of one channel half
  constexpr int DT = D / 16;      // 16-channel MFMA tiles
  constexpr int RB = 2 * D;       // bytes per V row in LDS
  constexpr int PP = SM::PP;
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef float f4 __attribute__((ext_vector_type(4)));
  typedef int v4i __attribute__((ext_vector_type(4)));
  __shared__ SM sm;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int split = blockIdx.x;
  const int bkv = blockIdx.y;
  const int b = bkv / h_kv, kvh = bkv % h_kv;
  const int j0 = blockIdx.z * G;
  const int ng = min(G, gsz - j0);

  for (int i = tid; i < G * D4; i += DEC_THREADS) {
    const int g = i / D4, c = i % D4;
    int val = 0;
    if (g < ng) {
      const int64_t hq = (int64_t)b * h_q + kvh * gsz + j0 + g;
      val = reinterpret_cast<const int*>(q + hq * D)[c];
    }
    sm.q[g][c] = val;
  }
  if (tid < G) {
    const int64_t hq = (int64_t)b * h_q + kvh * gsz + j0 + tid;
    sm.qs[tid] = tid < ng ? q_scale[hq] : 0.f;
  }
  // P rows of the unused head columns stay zero
  for (int i = lane; i < 16 * PP; i += 64) sm.t.p[wave][i] = 0;
  float cb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cb[i] = codebook[i];
  __syncthreads();

  const int col = lane & 15, g4 = lane >> 4;  // MFMA roles
  const int kh = lane >> 5, kr = lane & 31;   // dequantisation roles
  // Q^T (B operand of QK): head col, channels 64 s + 16 g4 .. +15
  v4i qb[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    qb[s] = col < G ? *reinterpret_cast<const v4i*>(&sm.q[col][16 * s + 4 * g4]) : v4i{0, 0, 0, 0};
  // (at least FLT_MIN: a masked key's -inf logit must stay -inf, never 0 * -inf)
  const float qsl = col < G ? fmaxf(sm.qs[col], 1.17549435e-38f) : 0.f;

  const int per = (n_len + n_splits - 1) / n_splits;
  const int n0 = split * per;
  // a context length above max_context_len (n_len) is read as max_context_len
  const int n1 = min(min(pg.ctx[b], n_len), n0 + per);
  const int32_t* btb = pg.bt + (int64_t)b * pg.maxb;

  // 32-byte chunk swizzle of V row r: 8 distinct values over the 16 rows one
  // transposed read touches (rows 8g + 0..3 and 8g + 4..7)
  auto vswz = [](int r) { return (r & 3) | (((r >> 3) & 1) << 2); };
  const int wsw = vswz(kr);
  // transposed read of lane (g4, j = col): rows 8 g4 + j / 4 (+4), channels 4 (j % 4)
  const int rr = 8 * g4 + (col >> 2);
  const int rsw = vswz(rr);
  const int rbase = rr * RB + 8 * (col & 3);
  uint16_t* vt = sm.t.v[wave];
  uint16_t* pt = sm.t.p[wave];
  float* kst = sm.t.ks[wave];

  // block-table entry of key lane + t (lanes past the split read key n0's)
  auto bt_entry = [&](int t) -> int {
    const int nn = t + lane < n1 ? t + lane : n0;
    return btb[pg.bs_sh >= 0 ? nn >> pg.bs_sh : nn / pg.bs];
  };
  // cache row of key lane + t (< 2^31: checked by the launcher)
  auto key_row = [&](int t, int blk) -> int {
    const int nn = t + lane < n1 ? t + lane : n0;
    const int off = pg.bs_sh >= 0 ? nn & (pg.bs - 1) : nn % pg.bs;
    return (blk * h_kv + kvh) * pg.bs + off;
  };
  // tile inputs (one register set, reloaded piece by piece after last use)
  v4i ka[4][KS];        // K: key 16 kb + col, channels 64 s + 16 g4 .. +15
  float ksv;            // k_scale of key lane
  float nrm[VB];        // norms of key lane
  uint2 cw[2][HW / 2];  // code bits of channel half kh of key 32 h + kr
  auto load_k = [&](int row) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int r = __shfl(row, 16 * kb + col, 64);
      const int8_t* kp = k + (int64_t)r * D + 16 * g4;
#pragma unroll
      for (int s = 0; s < KS; ++s) ka[kb][s] = *reinterpret_cast<const v4i*>(kp + 64 * s);
    }
    ksv = k_scale[row];
  };
  auto load_nrm = [&](int row) {
#pragma unroll
    for (int j = 0; j < VB; ++j) nrm[j] = vnorm[(int64_t)row * VB + j];
  };
  auto load_codes = [&](int row, int h) {
    const int r = __shfl(row, 32 * h + kr, 64);
    const uint2* cp = reinterpret_cast<const uint2*>(vpk + (int64_t)r * VW + kh * HW);
#pragma unroll
    for (int w = 0; w < HW / 2; ++w) cw[h][w] = cp[w];
  };

  float m_run = -INFINITY, l_lane = 0.f;  // head col
  f4 oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = f4{0.f, 0.f, 0.f, 0.f};

  constexpr int TSTEP = DEC_WAVES * DEC_TILE;
  int t0 = n0 + wave * DEC_TILE;
  int btn = 0;  // block-table entry of the next tile's key lane
  if (t0 < n1) {  // (an empty split has no valid key row to read)
    const int row = key_row(t0, bt_entry(t0));
    load_k(row);
    load_nrm(row);
    load_codes(row, 0);
    load_codes(row, 1);
    btn = bt_entry(t0 + TSTEP);
  }
  // The loads are unconditional inside the loop (n0 < n1 there, and lanes
  // past the split read key n0's row): loads under a branch would make the
  // compiler wait for all of them at the join.
  while (t0 < n1) {
    const int nrow = key_row(t0 + TSTEP, btn);
    kst[lane] = ksv;
    // ---- QK on the matrix core ----
    v4i sacc[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      sacc[kb] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        sacc[kb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka[kb][s], qb[s], sacc[kb], 0, 0, 0);
    }
    load_k(nrow);
    btn = bt_entry(t0 + 2 * TSTEP);
    // ---- value tables of key lane ----
    uint4 tbl[VB];
#pragma unroll
    for (int j = 0; j < VB; ++j) {
      // fp16 values of entries 0..7: the product rounded to fp32 first, then
      // to fp16. The empty asm keeps the fp32 product in a register:
      // otherwise the multiply and the conversion fuse into one
      // v_fma_mixlo_f16, which rounds the exact product once (a different
      // fp16 value when the fp32 product lands on an fp16 midpoint).
      float pr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pr[e] = cb[e] * nrm[j];
        asm volatile("" : "+v"(pr[e]));
      }
      uint32_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        h[e] = (uint32_t)f2h_bits(pr[2 * e]) | ((uint32_t)f2h_bits(pr[2 * e + 1]) << 16);
      tbl[j].x = __builtin_amdgcn_perm(h[1], h[0], 0x06040200u);  // low bytes of 0..3
      tbl[j].y = __builtin_amdgcn_perm(h[3], h[2], 0x06040200u);  // low bytes of 4..7
      tbl[j].z = __builtin_amdgcn_perm(h[1], h[0], 0x07050301u);  // high bytes of 0..3
      tbl[j].w = __builtin_amdgcn_perm(h[3], h[2], 0x07050301u);  // high bytes of 4..7
    }
    load_nrm(nrow);
    // tables of the dequantising lane's 128-channel block, both halves
    uint4 tv[2];
    {
      const uint4& tf = tbl[0];
      const uint4& ts = tbl[VB - 1];
      tv[0].x = swap32_lo(tf.x, ts.x); tv[1].x = swap32_hi(tf.x, ts.x);
      tv[0].y = swap32_lo(tf.y, ts.y); tv[1].y = swap32_hi(tf.y, ts.y);
      tv[0].z = swap32_lo(tf.z, ts.z); tv[1].z = swap32_hi(tf.z, ts.z);
      tv[0].w = swap32_lo(tf.w, ts.w); tv[1].w = swap32_hi(tf.w, ts.w);
    }
    // ---- softmax of head col over the tile ----
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float x[4][4];
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const float4 kv = *reinterpret_cast<const float4*>(kst + 16 * kb + 4 * g4);
      const float kk[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[kb][i] = (float)sacc[kb][i] * kk[i];
        mt = fmaxf(mt, x[kb][i]);
      }
    }
    if (t0 + DEC_TILE > n1) {  // the split's last tile: keys past it are masked
      mt = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (t0 + 16 * kb + 4 * g4 + i >= n1) x[kb][i] = -INFINITY;
          mt = fmaxf(mt, x[kb][i]);
        }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mn = fmaxf(m_run, mt * qsl);
    const float resc = __builtin_amdgcn_exp2f(m_run - mn);  // first tile: exp2(-inf) = 0
    m_run = mn;
    float ls = 0.f;
    uint32_t ph[4][2];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = __builtin_amdgcn_exp2f(fmaf(x[kb][i], qsl, -mn));  // masked key: -inf -> 0
        ls += p[i];
      }
      ph[kb][0] = (uint32_t)f2h_bits(p[0]) | ((uint32_t)f2h_bits(p[1]) << 16);
      ph[kb][1] = (uint32_t)f2h_bits(p[2]) | ((uint32_t)f2h_bits(p[3]) << 16);
    }
    l_lane = l_lane * resc + ls;
    if (col < G) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        *reinterpret_cast<uint2*>(pt + col * PP + 16 * kb + 4 * g4) = uint2{ph[kb][0], ph[kb][1]};
    }
    // rescale the accumulators only when some head's running max moved
    if (__builtin_amdgcn_ballot_w64(col < G && resc != 1.f)) {
#pragma unroll
      for (int t = 0; t < DT; ++t) oacc[t] *= resc;
    }

    // ---- PV, two 32-key halves ----
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      if (hf) __builtin_amdgcn_wave_barrier();  // half 0's tile reads are done
      uint32_t cc[HW];
#pragma unroll
      for (int w = 0; w < HW / 2; ++w) {
        cc[2 * w] = cw[hf][w].x;
        cc[2 * w + 1] = cw[hf][w].y;
      }
      load_codes(nrow, hf);
      // dequantise D/2 channels (D/16 groups of 8) of key row kr to LDS
#pragma unroll
      for (int gi = 0; gi < D / 16; ++gi) {
        const int bit = 24 * gi, w = bit >> 5, sh = bit & 31;
        const uint32_t xw = sh <= 8 ? (cc[w] >> sh)
                                    : __builtin_amdgcn_alignbit(cc[w + 1], cc[w], sh);
        const int c16 = kh * (D / 16) + gi;  // 16-byte chunk of the row
        const int off = kr * RB + ((((c16 >> 1) ^ wsw) << 1) | (c16 & 1)) * 16;
        *reinterpret_cast<uint4*>(reinterpret_cast<char*>(vt) + off) = lm3_lookup8(xw, tv[hf]);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // B = P^T: keys 32 hf + 8 g4 .. +7 of head col
      const h8 pb = *reinterpret_cast<const h8*>(pt + col * PP + 32 * hf + 8 * g4);
      const char* vbytes = reinterpret_cast<const char*>(vt);
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const char* a0 = vbytes + rbase + ((t ^ rsw) << 5);
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(a0));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(a0 + 4 * RB));
        typedef short v8s __attribute__((ext_vector_type(8)));
        const v8s both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        oacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, both), pb, oacc[t],
                                                         0, 0, 0);
      }
    }
    __builtin_amdgcn_wave_barrier();  // the wave's tile region is rewritten next tile
    t0 += TSTEP;
  }
  __syncthreads();  // every wave is done with the tile region (aliased below)

  // head col: l over the 4 lanes of the column
  l_lane += __shfl_xor(l_lane, 16, 64);
  l_lane += __shfl_xor(l_lane, 32, 64);
  if (g4 == 0 && col < G) {
    sm.r.m[wave][col] = m_run;
    sm.r.l[wave][col] = l_lane;
  }
  // accumulator lane (g4, col) holds channels 16 t + 4 g4 + i of head col
  if (col < G) {
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) sm.r.o[wave][col][16 * t + 4 * g4 + i] = oacc[t][i];
  }
  __syncthreads();

  for (int i = tid; i < G * D; i += DEC_THREADS) {
    const int g = i / D, d = i % D;
    if (g >= ng) continue;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < DEC_WAVES; ++w) mm = fmaxf(mm, sm.r.m[w][g]);
    float acc = 0.f, den = 0.f;
    if (mm != -INFINITY) {
#pragma unroll
      for (int w = 0; w < DEC_WAVES; ++w) {
        const float wt = exp2f(sm.r.m[w][g] - mm);
        acc += sm.r.o[w][g][d] * wt;
        den += sm.r.l[w][g] * wt;
      }
    }
    const int64_t hq = (int64_t)b * h_q + kvh * gsz + j0 + g;
    const int64_t orow = (int64_t)split * bhq + hq;
    o_part[orow * D + d] = acc;
    if (d == 0) {
      m_part[orow] = (mm == -INFINITY) ? DEC_NEG_INF : mm;
      l_part[orow] = den;
    }
  }
}

}  // namespace
}  // namespace sl8

// Auto split count of the paged decode (reference attn_paged_decode.cu:14-31):
// ~2048 (split, head) blocks, 48..256 keys per split, at most DEC_MAX_SPLITS.
extern "C" int sl8_paged_choose_num_splits(int64_t n_len_max, int64_t bhq) {
  if (n_len_max <= 0 || bhq <= 0) return 1;
  const int64_t s_occ = (2048 + bhq - 1) / bhq;
  const int64_t s_lo = (n_len_max + 255) / 256;
  int64_t s_hi = (n_len_max + 47) / 48;
  if (s_hi < 1) s_hi = 1;
  int64_t s = s_occ > s_lo ? s_occ : s_lo;
  if (s > s_hi) s = s_hi;
  if (s < 1) s = 1;
  if (s > DEC_MAX_SPLITS) s = DEC_MAX_SPLITS;
  return (int)s;
}

extern "C" int sl8_attn_paged_decode(const int8_t* q, const float* q_scale, const int8_t* k_cache,
                                     const float* k_scale, const int8_t* v_cache,
                                     const float* v_scale, const int32_t* block_table,
                                     const int32_t* context_lens, void* out, int64_t B,
                                     int64_t Hq, int64_t Hkv, int64_t D, int64_t num_blocks,
                                     int64_t block_size, int64_t max_blocks_per_seq,
                                     int64_t max_context_len, int64_t num_splits,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  SL8_CHECK_ARG(B >= 0 && Hq >= 0 && Hkv > 0 && num_blocks >= 0 && block_size > 0 &&
                    max_blocks_per_seq >= 0,
                "fni8 paged_decode: bad shape");
  SL8_CHECK_ARG(Hq % Hkv == 0, "fni8 paged_decode: H_q must be divisible by H_kv (GQA)");
  SL8_CHECK_ARG(D == 32 || D == 64 || D == 128 || D == 256,
                "fni8 paged_decode: head dim must be 32/64/128/256, got %lld", (long long)D);
  SL8_CHECK_ARG(max_context_len >= 0 && max_context_len <= max_blocks_per_seq * block_size,
                "fni8 paged_decode: max_context_len exceeds block_table capacity");
  SL8_CHECK_ARG(B * Hq < (1LL << 31) && num_blocks * Hkv * block_size < (1LL << 40) &&
                    max_context_len < (1LL << 31),
                "fni8 paged_decode: shape too large");
  const int64_t bhq = B * Hq;
  if (num_splits < 0) num_splits = sl8_paged_choose_num_splits(max_context_len, bhq);
  SL8_CHECK_ARG(num_splits >= 1 && num_splits <= DEC_MAX_SPLITS,
                "fni8 paged_decode: num_splits must be 1..%d, got %lld", DEC_MAX_SPLITS,
                (long long)num_splits);
  if (B == 0 || Hq == 0) return SL8_OK;
  SL8_CHECK_ARG(q && q_scale && block_table && context_lens && out &&
                    (num_blocks == 0 || (k_cache && k_scale && v_cache && v_scale)),
                "fni8 paged_decode: null pointer");
  SL8_CHECK_ARG(aligned(q, 16) && aligned(k_cache, 16) && aligned(v_cache, 16),
                "fni8 paged_decode: q/k_cache/v_cache must be 16-byte aligned");
  const size_t need = sl8_attn_int8_decode_workspace(B, Hq, D, num_splits);
  SL8_CHECK_ARG(workspace && workspace_bytes >= need && aligned(workspace, 16),
                "fni8 paged_decode: workspace needs %zu bytes", need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int ns = (int)num_splits, ibhq = (int)bhq, gsz = (int)(Hq / Hkv);
  const int G = group_width(gsz);
  float* op = static_cast<float*>(workspace);
  float* mp = op + (size_t)ns * ibhq * D;
  float* lp = mp + (size_t)ns * ibhq;
  const dim3 grid((unsigned)ns, (unsigned)(B * Hkv), (unsigned)((gsz + G - 1) / G));
  int bs_sh = 0;
  while ((1LL << bs_sh) < block_size) ++bs_sh;
  const bool pow2 = (1LL << bs_sh) == block_size;
  const int64_t cache_rows = num_blocks * Hkv * block_size;
  const PagedArgs pg{block_table, context_lens, (int)max_blocks_per_seq, (int)block_size, bs_sh,
                     (int)std::min<int64_t>(cache_rows, (int64_t)0x7fffffff)};
  const int nmax = (int)max_context_len;
  const int64_t per = (max_context_len + ns - 1) / ns;
  const bool stream_ok = D != 32 && pow2 && per / block_size + 2 <= DEC_BT_MAX &&
                         ((gsz == 2 && D == 128) || gsz == 4 || gsz == 8);
  // streaming tiles hold T = 32 (2 heads per KV head) or 16 keys; when blocks
  // and split boundaries are multiples of T, each tile sits in one block
  const int64_t tkeys = gsz == 2 ? 32 : 16;
  const bool aligned_tiles = block_size % tkeys == 0 && per % tkeys == 0 &&
                             cache_rows * D < (1LL << 31);
  if (stream_ok) {
    const dim3 g2((unsigned)ns, (unsigned)(B * Hkv));
#define SL8_PWAVE(DD, GS, NB)                                                                   \
    do {                                                                                         \
      if (aligned_tiles)                                                                         \
        decode_wave_kernel<DD, GS, NB, true, true, false, true><<<g2, DEC_THREADS, 0, st>>>(     \
            q, q_scale, k_cache, k_scale, v_cache, v_scale, op, mp, lp, nmax, ns, (int)Hq,       \
            (int)Hkv, ibhq, pg);                                                                 \
      else                                                                                       \
        decode_wave_kernel<DD, GS, NB, true, true><<<g2, DEC_THREADS, 0, st>>>(                  \
            q, q_scale, k_cache, k_scale, v_cache, v_scale, op, mp, lp, nmax, ns, (int)Hq,       \
            (int)Hkv, ibhq, pg);                                                                 \
    } while (0)
// D = 128: a two-stage ring (37 KB of LDS per workgroup, so 4 workgroups
// per CU instead of 2) measured 210 us against 227 us with three stages at
// config 3's shape with 16-key blocks scattered over the pool: more
// independent block streams in flight beat a deeper ring per wave.
#define SL8_PWAVE_D(GS)                        \
    if (D == 64) SL8_PWAVE(64, GS, 4);         \
    else if (D == 128) SL8_PWAVE(128, GS, 2);  \
    else SL8_PWAVE(256, GS, 3);
    switch (gsz) {
      case 2: SL8_PWAVE(128, 2, 3); break;
      case 4: SL8_PWAVE_D(4); break;
      default: SL8_PWAVE_D(8); break;
    }
#undef SL8_PWAVE_D
#undef SL8_PWAVE
  } else {
#define SL8_PAGED(DD)                                                                          \
    launch_d<DD, true, true>(G, grid, q, q_scale, k_cache, k_scale, v_cache, v_scale, op, mp, lp, \
                             nmax, ns, (int)Hq, (int)Hkv, gsz, ibhq, st, pg)
    if (D == 32) SL8_PAGED(32);
    else if (D == 64) SL8_PAGED(64);
    else if (D == 128) SL8_PAGED(128);
    else SL8_PAGED(256);
#undef SL8_PAGED
  }
  SL8_CHECK_LAUNCH("attn_paged_decode split");
  launch_combine((int)D, ibhq, st, op, mp, lp, static_cast<uint16_t*>(out), ns, ibhq);
  SL8_CHECK_LAUNCH("attn_paged_decode combine");
  return SL8_OK;
}

extern "C" int sl8_attn_paged_decode_k8v3(const int8_t* q, const float* q_scale,
                                          const int8_t* k_cache, const float* k_scale,
                                          const int32_t* v_packed, const float* v_norm,
                                          const float* v_codebook, const int32_t* block_table,
                                          const int32_t* context_lens, void* out, int64_t B,
                                          int64_t Hq, int64_t Hkv, int64_t D, int64_t num_blocks,
                                          int64_t block_size, int64_t max_blocks_per_seq,
                                          int64_t max_context_len, int64_t num_splits,
                                          void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  SL8_CHECK_ARG(B >= 0 && Hq >= 0 && Hkv > 0 && num_blocks >= 0 && block_size > 0 &&
                    max_blocks_per_seq >= 0,
                "fni8 paged_decode_k8v3: bad shape");
  SL8_CHECK_ARG(Hq % Hkv == 0, "fni8 paged_decode_k8v3: H_q must be divisible by H_kv (GQA)");
  SL8_CHECK_ARG(D == 128 || D == 256,
                "fni8 paged_decode_k8v3: lloydmax3 requires head dim 128 or 256, got %lld",
                (long long)D);
  SL8_CHECK_ARG(max_context_len >= 0 && max_context_len <= max_blocks_per_seq * block_size,
                "fni8 paged_decode_k8v3: max_context_len exceeds block_table capacity");
  SL8_CHECK_ARG(B * Hq < (1LL << 31) && num_blocks * Hkv * block_size < (1LL << 40) &&
                    max_context_len < (1LL << 31),
                "fni8 paged_decode_k8v3: shape too large");
  const int64_t bhq = B * Hq;
  if (num_splits < 0) num_splits = sl8_paged_choose_num_splits(max_context_len, bhq);
  SL8_CHECK_ARG(num_splits >= 1 && num_splits <= DEC_MAX_SPLITS,
                "fni8 paged_decode_k8v3: num_splits must be 1..%d, got %lld", DEC_MAX_SPLITS,
                (long long)num_splits);
  if (B == 0 || Hq == 0) return SL8_OK;
  SL8_CHECK_ARG(q && q_scale && block_table && context_lens && out && v_codebook &&
                    (num_blocks == 0 || (k_cache && k_scale && v_packed && v_norm)),
                "fni8 paged_decode_k8v3: null pointer");
  SL8_CHECK_ARG(num_blocks * Hkv * block_size < (1LL << 31),
                "fni8 paged_decode_k8v3: cache too large (rows must fit in 31 bits)");
  SL8_CHECK_ARG(aligned(q, 4) && aligned(k_cache, 16) && aligned(v_packed, 16),
                "fni8 paged_decode_k8v3: q must be 4-byte aligned, k_cache/v_packed 16-byte aligned");
  const size_t need = sl8_attn_int8_decode_workspace(B, Hq, D, num_splits);
  SL8_CHECK_ARG(workspace && workspace_bytes >= need && aligned(workspace, 16),
                "fni8 paged_decode_k8v3: workspace needs %zu bytes", need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int ns = (int)num_splits, ibhq = (int)bhq, gsz = (int)(Hq / Hkv);
  const int G = group_width(gsz);
  float* op = static_cast<float*>(workspace);
  float* mp = op + (size_t)ns * ibhq * D;
  float* lp = mp + (size_t)ns * ibhq;
  const dim3 grid((unsigned)ns, (unsigned)(B * Hkv), (unsigned)((gsz + G - 1) / G));
  int bs_sh = 0;
  while ((1LL << bs_sh) < block_size) ++bs_sh;
  if ((1LL << bs_sh) != block_size) bs_sh = -1;  // not a power of two: divide
  const PagedArgs pg{block_table, context_lens, (int)max_blocks_per_seq, (int)block_size, bs_sh, 0};
  const uint32_t* vp = reinterpret_cast<const uint32_t*>(v_packed);
#define SL8_K3(DD, GG)                                                                      \
  k8v3_split_kernel<DD, GG><<<grid, DEC_THREADS, 0, st>>>(                                  \
      q, q_scale, k_cache, k_scale, vp, v_norm, v_codebook, op, mp, lp, (int)max_context_len, \
      ns, (int)Hq, (int)Hkv, gsz, ibhq, pg)
#define SL8_K3D(DD)                     \
  switch (G) {                          \
    case 1: SL8_K3(DD, 1); break;       \
    case 2: SL8_K3(DD, 2); break;       \
    case 4: SL8_K3(DD, 4); break;       \
    default: SL8_K3(DD, 8); break;      \
  }
  if (D == 128) SL8_K3D(128)
  else SL8_K3D(256)
#undef SL8_K3D
#undef SL8_K3
  SL8_CHECK_LAUNCH("attn_paged_decode_k8v3 split");
  launch_combine((int)D, ibhq, st, op, mp, lp, static_cast<uint16_t*>(out), ns, ibhq);
  SL8_CHECK_LAUNCH("attn_paged_decode_k8v3 combine");
  return SL8_OK;
}

extern "C" int sl8_kv_write_paged(const void* k_new, const void* v_new, const int32_t* slot_mapping,
                                  int8_t* k_cache, float* k_scale, int8_t* v_cache, float* v_scale,
                                  int64_t B, int64_t Hkv, int64_t D, int64_t num_blocks,
                                  int64_t block_size, void* stream) {
  clear_error();
  SL8_CHECK_ARG(B >= 0 && Hkv > 0 && num_blocks >= 0 && block_size > 0,
                "fni8 kv_write_paged: bad shape");
  SL8_CHECK_ARG(D == 32 || D == 64 || D == 128 || D == 256,
                "fni8 kv_write_paged: head dim must be 32/64/128/256, got %lld", (long long)D);
  if (B == 0) return SL8_OK;
  SL8_CHECK_ARG(k_new && v_new && slot_mapping && k_cache && k_scale && v_cache && v_scale,
                "fni8 kv_write_paged: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(B * Hkv));
  const uint16_t* kn = static_cast<const uint16_t*>(k_new);
  const uint16_t* vn = static_cast<const uint16_t*>(v_new);
  if (D == 32) kv_write_paged_kernel<32><<<grid, 64, 0, st>>>(kn, vn, slot_mapping, k_cache, k_scale, v_cache, v_scale, (int)Hkv, (int)block_size);
  else if (D == 64) kv_write_paged_kernel<64><<<grid, 64, 0, st>>>(kn, vn, slot_mapping, k_cache, k_scale, v_cache, v_scale, (int)Hkv, (int)block_size);
  else if (D == 128) kv_write_paged_kernel<128><<<grid, 64, 0, st>>>(kn, vn, slot_mapping, k_cache, k_scale, v_cache, v_scale, (int)Hkv, (int)block_size);
  else kv_write_paged_kernel<256><<<grid, 64, 0, st>>>(kn, vn, slot_mapping, k_cache, k_scale, v_cache, v_scale, (int)Hkv, (int)block_size);
  SL8_CHECK_LAUNCH("kv_write_paged");
  return SL8_OK;
}
