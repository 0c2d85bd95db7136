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

#include "common.hpp"

namespace sl8 {
namespace {

constexpr int DEC_THREADS = 256;
constexpr int DEC_WAVES = 4;
constexpr int DEC_TILE = 64;
constexpr float DEC_NEG_INF = -1e30f;
constexpr int DEC_MAX_SPLITS = 256;

template <int D, int G>
struct DecSmem {
  int q[G][D / 4];                 // int8 Q, packed
  float qs[G];
  float p[DEC_WAVES][DEC_TILE][G];  // per-wave probabilities of the current tile
  float m[DEC_WAVES][G];
  float l[DEC_WAVES][G];
  float o[DEC_WAVES][G][D];
};

template <int D, int G>
__global__ void __launch_bounds__(DEC_THREADS)
decode_split_kernel(const int8_t* __restrict__ q, const float* __restrict__ q_scale,
                    const int8_t* __restrict__ k, const float* __restrict__ k_scale,
                    const uint16_t* __restrict__ v, float* __restrict__ o_part,
                    float* __restrict__ m_part, float* __restrict__ l_part, int n_len,
                    int n_splits, int h_q, int h_kv, int gsz, int bhq) {
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
  const int n1 = min(n_len, n0 + per);
  const int8_t* kb = k + (int64_t)bkv * n_len * D;
  const float* ksb = k_scale + (int64_t)bkv * n_len;
  const uint16_t* vb = v + (int64_t)bkv * n_len * D;

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
      const int4* kp = reinterpret_cast<const int4*>(kb + (int64_t)(valid ? n : n0) * D);
#pragma unroll
      for (int c = 0; c < D / 16; ++c) kr[c] = kp[c];
      const float ks = valid ? ksb[n] : 0.f;
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
        const uint4 vv = *reinterpret_cast<const uint4*>(vb + (int64_t)nn * D + dg * 8);
        float vf[8];
        vf[0] = h2f(vv.x & 0xFFFF); vf[1] = h2f(vv.x >> 16);
        vf[2] = h2f(vv.y & 0xFFFF); vf[3] = h2f(vv.y >> 16);
        vf[4] = h2f(vv.z & 0xFFFF); vf[5] = h2f(vv.z >> 16);
        vf[6] = h2f(vv.w & 0xFFFF); vf[7] = h2f(vv.w >> 16);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float p = sm.p[wave][kk][g];
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
    o_part[row * D + d] = acc;
    if (d == 0) {
      m_part[row] = (mm == -INFINITY) ? DEC_NEG_INF : mm;
      l_part[row] = den;
    }
  }
}

// One block per query head; thread = channel.
__global__ void decode_combine_kernel(const float* __restrict__ o_part,
                                      const float* __restrict__ m_part,
                                      const float* __restrict__ l_part,
                                      uint16_t* __restrict__ out, int n_splits, int bhq, int D) {
  const int64_t hq = blockIdx.x;
  float gm = DEC_NEG_INF;
  for (int s = 0; s < n_splits; ++s) gm = fmaxf(gm, m_part[(int64_t)s * bhq + hq]);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float acc = 0.f, den = 0.f;
    for (int s = 0; s < n_splits; ++s) {
      const int64_t row = (int64_t)s * bhq + hq;
      const float ms = m_part[row];
      if (ms == DEC_NEG_INF) continue;
      const float wt = exp2f(ms - gm);
      den += l_part[row] * wt;
      acc += o_part[row * D + d] * wt;
    }
    out[hq * D + d] = f2h_bits(den > 0.f ? acc / den : 0.f);
  }
}

template <int D, int G>
void launch_split(dim3 grid, const int8_t* q, const float* qs, const int8_t* k, const float* ks,
                  const uint16_t* v, float* op, float* mp, float* lp, int N, int ns, int hq,
                  int hkv, int gsz, int bhq, hipStream_t st) {
  decode_split_kernel<D, G><<<grid, DEC_THREADS, 0, st>>>(q, qs, k, ks, v, op, mp, lp, N, ns, hq,
                                                          hkv, gsz, bhq);
}

template <int D>
void launch_d(int G, dim3 grid, const int8_t* q, const float* qs, const int8_t* k,
              const float* ks, const uint16_t* v, float* op, float* mp, float* lp, int N, int ns,
              int hq, int hkv, int gsz, int bhq, hipStream_t st) {
  switch (G) {
    case 1: launch_split<D, 1>(grid, q, qs, k, ks, v, op, mp, lp, N, ns, hq, hkv, gsz, bhq, st); break;
    case 2: launch_split<D, 2>(grid, q, qs, k, ks, v, op, mp, lp, N, ns, hq, hkv, gsz, bhq, st); break;
    case 4: launch_split<D, 4>(grid, q, qs, k, ks, v, op, mp, lp, N, ns, hq, hkv, gsz, bhq, st); break;
    default: launch_split<D, 8>(grid, q, qs, k, ks, v, op, mp, lp, N, ns, hq, hkv, gsz, bhq, st); break;
  }
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

extern "C" int sl8_attn_int8_decode(const int8_t* q, const float* q_scale, const int8_t* k,
                                    const float* k_scale, const void* v, void* out, int64_t B,
                                    int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                                    int64_t num_splits, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  clear_error();
  SL8_CHECK_ARG(B >= 0 && Hq >= 0 && Hkv > 0 && N >= 0, "fni8 decode: bad shape");
  SL8_CHECK_ARG(Hq % Hkv == 0, "fni8 decode: H_q must be divisible by H_kv (GQA)");
  SL8_CHECK_ARG(D == 64 || D == 128 || D == 256, "fni8 decode: head dim must be 64/128/256, got %lld",
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
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int ns = (int)num_splits, bhq = (int)(B * Hq), gsz = (int)(Hq / Hkv);
  const int G = group_width(gsz);
  float* op = static_cast<float*>(workspace);
  float* mp = op + (size_t)ns * bhq * D;
  float* lp = mp + (size_t)ns * bhq;
  const dim3 grid((unsigned)ns, (unsigned)(B * Hkv), (unsigned)((gsz + G - 1) / G));
  const uint16_t* vp = static_cast<const uint16_t*>(v);
  switch (D) {
    case 64: launch_d<64>(G, grid, q, q_scale, k, k_scale, vp, op, mp, lp, (int)N, ns, (int)Hq, (int)Hkv, gsz, bhq, st); break;
    case 128: launch_d<128>(G, grid, q, q_scale, k, k_scale, vp, op, mp, lp, (int)N, ns, (int)Hq, (int)Hkv, gsz, bhq, st); break;
    default: launch_d<256>(G, grid, q, q_scale, k, k_scale, vp, op, mp, lp, (int)N, ns, (int)Hq, (int)Hkv, gsz, bhq, st); break;
  }
  SL8_CHECK_LAUNCH("attn_int8_decode split");
  decode_combine_kernel<<<bhq, (unsigned)(D < 256 ? D : 256), 0, st>>>(
      op, mp, lp, static_cast<uint16_t*>(out), ns, bhq, (int)D);
  SL8_CHECK_LAUNCH("attn_int8_decode combine");
  return SL8_OK;
}
