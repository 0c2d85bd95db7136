// Full-W8A8 prefill attention for gfx950.
//
// per_warp_quant = 1 (the reference default) runs on the prefill pipeline of
// attn_fwd.hip (attn_fwd_wide_kernel, W8 = true): int8 Q.K^T on the int8
// MFMA, P codes re-quantised per 32-key half and fed to the bf16 MFMA as
// code * per-row factor against int8 V held exactly in bf16 (w8a8_wide_launch).
// This file holds the kernel with int8 Q.K^T and int8 P.V, both on the int8
// MFMA (v_mfma_i32_32x32x32_i8): per_warp_quant = 0 (one P scale per 64-key
// tile) and per_warp_quant = 2, the reference's per-warp arithmetic exactly
// (one P scale per 32-key half, an exact int32 P.V per half scaled in fp32,
// the running max updated every tile) at about twice the time of mode 1.
//
// Semantics follow the reference (csrc/include/attn_w8a8_fwd.cuh:30-235):
//   logits and the online softmax as attn_int8_fwd, over 64-key tiles, with
//   the running max updated every tile (m_new = max(m, tile max));
//   P of each tile re-quantised to int8: p_scale = max(pmax * (1/127), 2e-38),
//   code = rint(p * (1/p_scale)); pmax is taken per query row over the whole
//   64-key tile, or (per_warp_quant) separately for each 32-key half;
//   O += int32(P_i8 . V_i8) * p_scale; the denominator sums the unquantised p;
//   V is int8 with a per-channel scale applied once in the epilogue (it does
//   not depend on the key, so it factors out of every sum);
//   causal: query i sees keys <= i + causal_diag; output fp16.
//
// Layout. As in attn_fwd.hip the scores are computed transposed
// (S^T = K . Q^T) so that a lane holds one query and 16 keys of each 32-key
// half; those 16 probabilities are exactly the lane's 16 int8 B-operand
// slots of O^T = V^T . P^T, so P is quantised and packed in registers. V^T is
// staged once per call into the workspace ([B*Hkv][D][Npad] int8), with the
// keys of each 32-key group stored in the order the A operand consumes them.

#include "attn_common.hpp"

namespace sl8 {
namespace {

constexpr int WT = 256;  // threads per workgroup
constexpr int WBM = 128; // queries per workgroup
constexpr int WBN = 64;  // keys per tile

// storage position p (0..31) inside a 32-key group -> key index
__host__ __device__ __forceinline__ int vt8_key(int p) {
  return 8 * ((p & 15) >> 2) + 4 * (p >> 4) + (p & 3);
}

template <int D>
__global__ void __launch_bounds__(256)
v8_transpose_kernel(const int8_t* __restrict__ v, int8_t* __restrict__ vt, int N, int Npad) {
  __shared__ int8_t tile[WBN][D + 4];
  const int64_t bh = blockIdx.y;
  const int n0 = blockIdx.x * WBN;
  const int8_t* src = v + bh * (int64_t)N * D;
  for (int i = threadIdx.x; i < WBN * D / 16; i += 256) {
    const int r = i / (D / 16), c = (i % (D / 16)) * 16;
    uint4 val = {0, 0, 0, 0};
    if (n0 + r < N) val = *reinterpret_cast<const uint4*>(src + (int64_t)(n0 + r) * D + c);
    const uint32_t w[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      *reinterpret_cast<uint32_t*>(&tile[r][c + 4 * e]) = w[e];
  }
  __syncthreads();
  int8_t* dst = vt + bh * (int64_t)D * Npad + n0;
  for (int i = threadIdx.x; i < D * (WBN / 4); i += 256) {
    const int d = i / (WBN / 4), p = (i % (WBN / 4)) * 4;  // positions p..p+3
    const int k0 = (p & ~31) + vt8_key(p & 31);            // 4 consecutive keys
    const uint32_t w = (uint8_t)tile[k0][d] | ((uint32_t)(uint8_t)tile[k0 + 1][d] << 8) |
                       ((uint32_t)(uint8_t)tile[k0 + 2][d] << 16) |
                       ((uint32_t)(uint8_t)tile[k0 + 3][d] << 24);
    *reinterpret_cast<uint32_t*>(dst + (int64_t)d * Npad + p) = w;
  }
}

struct W8Args {
  const int8_t* q;
  const float* qs;
  const int8_t* k;
  const float* ks;
  const int8_t* vt;
  const float* vs;
  uint16_t* out;
  int M, N, Npad, Hq, Hkv, nqb, causal_diag;
  int xcd_map;
  int dout;  // output row length (< D when the operands are zero-padded)
};

__device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d) {
  return (uint32_t)(uint8_t)(int)a | ((uint32_t)(uint8_t)(int)b << 8) |
         ((uint32_t)(uint8_t)(int)c << 16) | ((uint32_t)(uint8_t)(int)d << 24);
}

template <int D, bool CAUSAL, bool PER_WARP>
__global__ void __launch_bounds__(WT, (D <= 128 ? 2 : 1))
attn_w8a8_kernel(const W8Args a) {
  constexpr int DC = D / 32;
  constexpr int KCPR = D / 16;                 // 16-B chunks per K row
  // LDS has 64 four-byte banks: 16 lanes of a 16-byte read touch 16
  // consecutive tile rows, so chunks are XOR-swizzled with the row index above
  // the rows sharing one 256-byte bank line (K rows: D bytes; V^T rows: 64).
  constexpr int KSW = KCPR - 1;
  constexpr int KSH = D == 64 ? 2 : (D == 128 ? 1 : 0);
  constexpr int KCH = WBN * D / 16 / WT;       // K chunks per thread
  constexpr int VCH = D * WBN / 16 / WT;       // V^T chunks per thread
  static_assert(KCH >= 1 && VCH >= 1, "tile copy covers D >= 64");
  __shared__ __attribute__((aligned(16))) int8_t sm_k0[WBN * D];
  __shared__ __attribute__((aligned(16))) int8_t sm_k1[WBN * D];
  __shared__ __attribute__((aligned(16))) int8_t sm_v0[D * WBN];
  __shared__ __attribute__((aligned(16))) int8_t sm_v1[D * WBN];
  __shared__ __attribute__((aligned(16))) float sm_s0[WBN];
  __shared__ __attribute__((aligned(16))) float sm_s1[WBN];

  const int nslot = CAUSAL ? (a.nqb + 1) / 2 : a.nqb;
  int bh, slot;
  attn_block_coords(a.Hq, a.Hkv, nslot, a.xcd_map, bh, slot);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  const int gsz = a.Hq / a.Hkv;
  const int b = bh / a.Hq, hq = bh % a.Hq;
  const int64_t bkv = (int64_t)b * a.Hkv + hq / gsz;
  const int M = a.M, N = a.N;
  const int diag = CAUSAL ? a.causal_diag : 0;

  const int8_t* kb = a.k + bkv * (int64_t)N * D;
  const float* ksb = a.ks + bkv * (int64_t)N;
  const int8_t* vtb = a.vt + bkv * (int64_t)D * a.Npad;

  int koff[DC], voff[2];
#pragma unroll
  for (int ch = 0; ch < DC; ++ch) koff[ch] = ((2 * ch + h) ^ ((l32 >> KSH) & KSW)) * 16;
#pragma unroll
  for (int st = 0; st < 2; ++st) voff[st] = ((2 * st + h) ^ ((l32 >> 2) & 3)) * 16;

  int qbs[2] = {a.nqb - 1 - slot, slot};
  const int npass = (CAUSAL && qbs[1] != qbs[0]) ? 2 : 1;

  for (int pass = 0; pass < npass; ++pass) {
    const int m_blk = qbs[pass] * WBM;
    const int mq = m_blk + wave * 32 + l32;
    const bool m_ok = mq < M;
    const int qpos = mq + diag;
    v4i qop[DC];
    {
      const int8_t* qrow = a.q + ((int64_t)bh * M + (m_ok ? mq : M - 1)) * D + 16 * h;
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        qop[c] = *reinterpret_cast<const v4i*>(qrow + 32 * c);
        if (!m_ok) qop[c] = v4i{0, 0, 0, 0};
      }
    }
    const float qsc = m_ok ? a.qs[(int64_t)bh * M + mq] : 1.f;

    int n_end = N;
    if (CAUSAL) n_end = max(0, min(N, m_blk + WBM + diag));
    const int ntiles = (n_end + WBN - 1) / WBN;
    const int wq_lo = m_blk + wave * 32 + diag, wq_hi = wq_lo + 31;

    auto load_tile = [&](int n0, int8_t* kd, int8_t* vd, float* sd) {
#pragma unroll
      for (int i = 0; i < KCH; ++i) {
        const int s = i * WT + tid;
        const int row = s / KCPR;
        const int c = (s % KCPR) ^ ((row >> KSH) & KSW);
        dma16_to_lds(kb + (int64_t)min(n0 + row, N - 1) * D + 16 * c, kd + (i * WT + wave * 64) * 16);
      }
#pragma unroll
      for (int i = 0; i < VCH; ++i) {
        const int s = i * WT + tid;
        const int row = s / 4;
        const int c = (s % 4) ^ ((row >> 2) & 3);
        dma16_to_lds(vtb + (int64_t)row * a.Npad + n0 + 16 * c, vd + (i * WT + wave * 64) * 16);
      }
      if (wave == 0) dma4_to_lds(ksb + min(n0 + lane, N - 1), sd);
    };

    v16f oacc[DC];
#pragma unroll
    for (int t = 0; t < DC; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[t][r] = 0.f;
    float m_run = -INFINITY, l_lane = 0.f;

    if (ntiles > 0) load_tile(0, sm_k0, sm_v0, sm_s0);
    wait_dma();
    __syncthreads();

    auto body = [&](int j, const int8_t* kc, const int8_t* vc, const float* scur, int8_t* kn,
                    int8_t* vn, float* snext) {
      const int n0 = j * WBN;
      if (j + 1 < ntiles) load_tile(n0 + WBN, kn, vn, snext);
      const bool live = !(CAUSAL && n0 > wq_hi);
      if (live) {
        v16i s0, s1;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s0[r] = 0;
          s1[r] = 0;
        }
        const int8_t* kt = kc + l32 * D;
#pragma unroll
        for (int ch = 0; ch < DC; ++ch) {
          const v4i k0 = *reinterpret_cast<const v4i*>(kt + koff[ch]);
          const v4i k1 = *reinterpret_cast<const v4i*>(kt + 32 * D + koff[ch]);
          s0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k0, qop[ch], s0, 0, 0, 0);
          s1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k1, qop[ch], s1, 0, 0, 0);
        }
        float t[32];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 ka = *reinterpret_cast<const float4*>(scur + 8 * g + 4 * h);
          const float4 kc4 = *reinterpret_cast<const float4*>(scur + 32 + 8 * g + 4 * h);
          t[4 * g + 0] = ((float)s0[4 * g + 0] * qsc) * ka.x;
          t[4 * g + 1] = ((float)s0[4 * g + 1] * qsc) * ka.y;
          t[4 * g + 2] = ((float)s0[4 * g + 2] * qsc) * ka.z;
          t[4 * g + 3] = ((float)s0[4 * g + 3] * qsc) * ka.w;
          t[16 + 4 * g + 0] = ((float)s1[4 * g + 0] * qsc) * kc4.x;
          t[16 + 4 * g + 1] = ((float)s1[4 * g + 1] * qsc) * kc4.y;
          t[16 + 4 * g + 2] = ((float)s1[4 * g + 2] * qsc) * kc4.z;
          t[16 + 4 * g + 3] = ((float)s1[4 * g + 3] * qsc) * kc4.w;
        }
        if ((n0 + WBN > N) || (CAUSAL && n0 + WBN - 1 > wq_lo)) {
#pragma unroll
          for (int e = 0; e < 32; ++e) {
            const int n = n0 + 32 * (e >> 4) + 8 * ((e & 15) >> 2) + 4 * h + (e & 3);
            bool ok = n < N;
            if (CAUSAL) ok = ok && n <= qpos;
            t[e] = ok ? t[e] : -INFINITY;
          }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int e = 0; e < 32; ++e) tmax = fmaxf(tmax, t[e]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m_run, tmax);
        const float resc =
            (m_run == -INFINITY || m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
        const float msub = (m_new == -INFINITY) ? 0.f : m_new;
        float psum = 0.f, pm0 = 0.f, pm1 = 0.f;
#pragma unroll
        for (int e = 0; e < 32; ++e) {
          const float p = __builtin_amdgcn_exp2f(t[e] - msub);  // -inf -> 0
          t[e] = p;
          psum += p;
          if (e < 16) pm0 = fmaxf(pm0, p);
          else pm1 = fmaxf(pm1, p);
        }
        pm0 = fmaxf(pm0, __shfl_xor(pm0, 32, 64));
        pm1 = fmaxf(pm1, __shfl_xor(pm1, 32, 64));
        if (!PER_WARP) {
          pm0 = fmaxf(pm0, pm1);
          pm1 = pm0;
        }
        const float ps0 = fmaxf(pm0 * (1.0f / 127.0f), 2e-38f);
        const float ps1 = fmaxf(pm1 * (1.0f / 127.0f), 2e-38f);
        const float inv0 = 1.0f / ps0, inv1 = 1.0f / ps1;
        v4i pq0, pq1;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          pq0[w] = (int)pack4(rintf(t[4 * w] * inv0), rintf(t[4 * w + 1] * inv0),
                              rintf(t[4 * w + 2] * inv0), rintf(t[4 * w + 3] * inv0));
          pq1[w] = (int)pack4(rintf(t[16 + 4 * w] * inv1), rintf(t[16 + 4 * w + 1] * inv1),
                              rintf(t[16 + 4 * w + 2] * inv1), rintf(t[16 + 4 * w + 3] * inv1));
        }
        l_lane = l_lane * resc + psum;
        m_run = m_new;
        if (m_new != -INFINITY) {
          const int8_t* vrow = vc + l32 * WBN;
#pragma unroll
          for (int tt = 0; tt < DC; ++tt) {
            const v4i va = *reinterpret_cast<const v4i*>(vrow + 32 * tt * WBN + voff[0]);
            const v4i vb = *reinterpret_cast<const v4i*>(vrow + 32 * tt * WBN + voff[1]);
            v16i z;
#pragma unroll
            for (int r = 0; r < 16; ++r) z[r] = 0;
            if (PER_WARP) {
              const v16i c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(va, pq0, z, 0, 0, 0);
              const v16i c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(vb, pq1, z, 0, 0, 0);
#pragma unroll
              for (int r = 0; r < 16; ++r)
                oacc[tt][r] = oacc[tt][r] * resc + ((float)c0[r] * ps0 + (float)c1[r] * ps1);
            } else {
              v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(va, pq0, z, 0, 0, 0);
              c = __builtin_amdgcn_mfma_i32_32x32x32_i8(vb, pq1, c, 0, 0, 0);
#pragma unroll
              for (int r = 0; r < 16; ++r) oacc[tt][r] = oacc[tt][r] * resc + (float)c[r] * ps0;
            }
          }
        }
      }
      wait_dma();
      __syncthreads();
    };

    for (int j = 0; j < ntiles; j += 2) {
      body(j, sm_k0, sm_v0, sm_s0, sm_k1, sm_v1, sm_s1);
      if (j + 1 < ntiles) body(j + 1, sm_k1, sm_v1, sm_s1, sm_k0, sm_v0, sm_s0);
    }

    const float l = l_lane + __shfl_xor(l_lane, 32, 64);
    if (m_ok) {
      const float inv = (l > 0.f) ? 1.f / l : 0.f;
      const float* vs = a.vs + bkv * D;
      uint16_t* orow = a.out + ((int64_t)bh * M + mq) * a.dout;
#pragma unroll
      for (int tt = 0; tt < DC; ++tt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = 32 * tt + 8 * g + 4 * h;
          if (d0 >= a.dout) continue;  // zero-padded channels
          const float4 sc = *reinterpret_cast<const float4*>(vs + d0);
          uint2 pk;
          pk.x = f2h_bits(oacc[tt][4 * g + 0] * sc.x * inv) |
                 ((uint32_t)f2h_bits(oacc[tt][4 * g + 1] * sc.y * inv) << 16);
          pk.y = f2h_bits(oacc[tt][4 * g + 2] * sc.z * inv) |
                 ((uint32_t)f2h_bits(oacc[tt][4 * g + 3] * sc.w * inv) << 16);
          *reinterpret_cast<uint2*>(orow + d0) = pk;
        }
    }
    __syncthreads();  // the next pass refills the tile buffers
  }
}

int64_t npad8(int64_t N) { return (N + WBN - 1) / WBN * WBN; }

template <int D, bool CAUSAL>
void launch_w8(const W8Args& a, int grid, bool per_warp, hipStream_t st) {
  if (per_warp) attn_w8a8_kernel<D, CAUSAL, true><<<grid, WT, 0, st>>>(a);
  else attn_w8a8_kernel<D, CAUSAL, false><<<grid, WT, 0, st>>>(a);
}

template <int D>
void launch_w8_d(const W8Args& a, int grid, bool causal, bool per_warp, hipStream_t st) {
  if (causal) launch_w8<D, true>(a, grid, per_warp, st);
  else launch_w8<D, false>(a, grid, per_warp, st);
}

}  // namespace

// per-warp quantisation runs on the prefill pipeline of attn_fwd.hip, which
// also pads head dim 32 to 64 (zero channels; see padded_head_dim there)
size_t w8a8_wide_workspace(int64_t B, int64_t Hkv, int64_t N, int64_t D);
size_t w8a8_pad_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t M, int64_t N, int64_t D);
int w8a8_pad_operands(const int8_t*& q, const int8_t*& k, const int8_t*& v, const float*& vs,
                      int64_t B, int64_t Hq, int64_t Hkv, int64_t M, int64_t N, int64_t D,
                      void*& ws, hipStream_t st);
int w8a8_wide_launch(const int8_t* q, const float* q_scale, const int8_t* k, const float* k_scale,
                     const int8_t* v, const float* v_scale, void* out, int64_t B, int64_t Hq,
                     int64_t Hkv, int64_t M, int64_t N, int64_t D, int64_t dout, bool causal,
                     int64_t causal_diag, void* vt_ws, hipStream_t st);

}  // namespace sl8

using namespace sl8;

extern "C" size_t sl8_attn_w8a8_fwd_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t M,
                                               int64_t N, int64_t D) {
  if (B <= 0 || Hkv <= 0 || D <= 0) return 0;
  const size_t pad = w8a8_pad_workspace(B, Hq, Hkv, M, N, D);
  if (N <= 0) return pad;
  // the larger of the two layouts: bf16 V^T (per-warp quantisation) and the
  // int8 V^T of the per-tile kernel, after the zero-padded operands (head dim 32)
  const int64_t DP = D == 32 ? 64 : D;
  const size_t i8 = (size_t)(B * Hkv * DP * npad8(N));
  const size_t f16 = w8a8_wide_workspace(B, Hkv, N, D);
  return pad + (f16 > i8 ? f16 : i8);
}

extern "C" int sl8_attn_w8a8_fwd(const int8_t* q, const float* q_scale, const int8_t* k,
                                 const float* k_scale, const int8_t* v, const float* v_scale,
                                 void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t M,
                                 int64_t N, int64_t D, int causal, int64_t causal_diag,
                                 int per_warp_quant, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  clear_error();
  SL8_CHECK_ARG(B >= 0 && Hq >= 0 && Hkv > 0 && M >= 0 && N >= 0, "fni8: bad shape");
  SL8_CHECK_ARG(Hq % Hkv == 0, "fni8: H_q must be divisible by H_kv (GQA)");
  SL8_CHECK_ARG(D == 32 || D == 64 || D == 128 || D == 256,
                "fni8: head dim must be 32/64/128/256, got %lld", (long long)D);
  SL8_CHECK_ARG(M < (1 << 30) && N < (1 << 30) && B * Hq < (1 << 24), "fni8: shape too large");
  SL8_CHECK_ARG(causal_diag > -(1LL << 30) && causal_diag < (1LL << 30), "fni8: bad causal_diag");
  if (B == 0 || Hq == 0 || M == 0) return SL8_OK;
  SL8_CHECK_ARG(q && q_scale && v_scale && out && (N == 0 || (k && k_scale && v)),
                "fni8: null pointer");
  SL8_CHECK_ARG(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(out, 16) &&
                    aligned(v_scale, 16),
                "fni8: q/k/v/v_scale/out must be 16-byte aligned");
  const size_t need = sl8_attn_w8a8_fwd_workspace(B, Hq, Hkv, M, N, D);
  SL8_CHECK_ARG(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 16)),
                "fni8: attn_w8a8_fwd workspace needs %zu bytes", need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t dout = D;
  if (D == 32) {
    // zero-padded to 64 channels: identical scores, zero output channels 32..63
    const int rc = w8a8_pad_operands(q, k, v, v_scale, B, Hq, Hkv, M, N, D, workspace, st);
    if (rc) return rc;
    D = 64;
  }
  SL8_CHECK_ARG(per_warp_quant >= 0 && per_warp_quant <= 2,
                "fni8: per_warp_quant must be 0 (per tile), 1 (per warp) or 2 (per warp, exact int32 PV)");
  if (per_warp_quant == 1)
    return w8a8_wide_launch(q, q_scale, k, k_scale, v, v_scale, out, B, Hq, Hkv, M, N, D, dout,
                            causal != 0, causal_diag, workspace, st);
  const int64_t Npad = npad8(N);
  if (N > 0) {
    const dim3 g((unsigned)(Npad / WBN), (unsigned)(B * Hkv));
    int8_t* vt = static_cast<int8_t*>(workspace);
    if (D == 64) v8_transpose_kernel<64><<<g, 256, 0, st>>>(v, vt, (int)N, (int)Npad);
    else if (D == 128) v8_transpose_kernel<128><<<g, 256, 0, st>>>(v, vt, (int)N, (int)Npad);
    else v8_transpose_kernel<256><<<g, 256, 0, st>>>(v, vt, (int)N, (int)Npad);
    SL8_CHECK_LAUNCH("attn_w8a8_fwd v transpose");
  }
  W8Args a{};
  a.q = q; a.qs = q_scale; a.k = k; a.ks = k_scale;
  a.vt = static_cast<const int8_t*>(workspace);
  a.vs = v_scale;
  a.out = static_cast<uint16_t*>(out);
  a.dout = (int)dout;
  a.M = (int)M; a.N = (int)N; a.Npad = (int)Npad; a.Hq = (int)Hq; a.Hkv = (int)Hkv;
  a.nqb = (int)((M + WBM - 1) / WBM);
  a.causal_diag = (int)causal_diag;
  const bool c = causal != 0, pw = per_warp_quant == 2;
  const int nslot = c ? (a.nqb + 1) / 2 : a.nqb;
  a.xcd_map = xcd_mode(B * Hkv, Hq / Hkv, nslot);
  const int grid = (int)(B * Hq * nslot);
  if (D == 64) launch_w8_d<64>(a, grid, c, pw, st);
  else if (D == 128) launch_w8_d<128>(a, grid, c, pw, st);
  else launch_w8_d<256>(a, grid, c, pw, st);
  SL8_CHECK_LAUNCH("attn_w8a8_fwd");
  return SL8_OK;
}
