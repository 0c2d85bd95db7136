// Prefill FlashAttention-2 for gfx950: int8 Q.K^T on MFMA, fp32 exp2-domain
// online softmax, fp16/bf16 P.V on MFMA.
//
// Semantics follow the reference (csrc/include/attn_int8_fwd.cuh:47-209):
//   logit  = ((float)<q_i8, k_i8> * q_scale[m]) * k_scale[n]   (exp2 domain)
//   causal = bottom-right aligned: query m sees keys n <= m + N - M
//   window = window_left >= 0 also requires n > m + N - M - window_left
//            (position m itself when not causal)
//   out    = sum_n 2^(s - max) v_n / sum_n 2^(s - max); a row with no visible
//            key is 0 and its LSE -inf; LSE = max*ln2 + ln(l).
//   GQA: query head h reads K/V head h / (Hq/Hkv).
//
// Work decomposition (attn_fwd_wide_kernel, the one kernel; its DUMP
// instantiation stores the int32 scores for the bit-exactness test): a wave
// owns 32 queries for the whole key loop, a workgroup 4 or 8 waves; 64-key K,
// k_scale and V tiles are copied global -> LDS one tile ahead and shared by
// the waves.
//
// The scores are computed transposed, S^T = K . Q^T, with
// v_mfma_i32_32x32x32_i8 (A = 32 keys x 32 channels from LDS, B = the wave's
// 32 queries x 32 channels held in registers). In the 32x32 accumulator
// layout a lane then holds one query (lane % 32) and 16 of the keys, which is
// exactly the B-operand layout of the next product O^T = V^T . P^T
// (v_mfma_f32_32x32x16_f16/bf16): P never leaves registers. The 8 keys a lane
// feeds per 16-key MFMA step are {4h..4h+3, 8+4h..8+4h+3} (h = lane / 32);
// the matching V^T operand is read from V's natural [key][D] layout in LDS
// with ds_read_b64_tr_b16 (two transposing reads per step), so V is used in
// place: no transpose pass, no workspace.
//
// Scheduling: workgroups are issued heaviest-first (causal), and, when the
// KV-head count is a multiple of 8, all query heads of one KV head go to the
// same XCD so its K/V tiles stay in that XCD's L2.

#include <algorithm>
#include <climits>

#include "attn_common.hpp"

namespace sl8 {
namespace {

constexpr int BN = 64;   // keys per tile
constexpr float LN2F = 0.6931471805599453f;
// Seeded QK accumulator of the D = 128 straight-line path: the int8 MFMA
// starts from the bit pattern of C0 = 1/(2 pi) (0x3E22F983, an inline
// constant of the MFMA's C operand, so no register has to be set), so the
// accumulator holds the integer C0BITS + acc. C0 lies in the binade
// [2^-3, 2^-2), whose float spacing is 2^-26, 2,292,099 steps above its
// lower end and 6,096,509 below its upper end: for |acc| <= 128 * 128^2 =
// 2,097,152 (D <= 128, any int8 codes) the bits read as the float
// C0 + acc * 2^-26 exactly, so no int -> float conversion is needed:
//   w = fma(f, q_scale * 2^26, -rn(C0 * q_scale * 2^26)) = q_scale * (acc + d),
//   |d| <= 2^-24 * C0 * 2^26 * (1 + 2^-23) ~ 0.64 (the rounding of the constant),
// and then x = fma(w, k_scale, -m): the exp2 argument in two fmas.
constexpr int C0BITS = 0x3E22F983;
constexpr float C0F = 0.15915494309189535f;  // the float with bits C0BITS
#ifndef SL8_W8_LAZY
#define SL8_W8_LAZY 1
#endif
// W8A8 reference point: set by the row's first visible half and raised
// lazily (see half_probs_w8) when a half's max exceeds it by more than the
// launch's w8_excess: P = code * 2^(max_half - m) / 127 then stays below
// 2^w8_excess, and with |V code| <= 127 the fp32 O and l sums over N keys
// stay below 2^(w8_excess + 7 + log2 N) <= 2^120 (w8_excess_for()).
constexpr bool W8_LAZY = SL8_W8_LAZY;


// W8A8 variant: int8 V -> bf16 V^T [BHkv][D][Npad] (Npad = N rounded up to 64,
// zero padded). Inside each 16-key group the keys are stored with bits 2 and 3
// of the index swapped, so the 8 keys {4h..4h+3, 8+4h..8+4h+3} a lane feeds
// per 16-key PV step are one 16-byte read. The per-warp W8A8 kernel reads V^T
// with plain 16-byte LDS reads: at D = 256 and one wave per SIMD its PV step
// is LDS-issue bound, where the two transposing reads per operand of the
// in-place layout cost 12% of the kernel time.
__host__ __device__ __forceinline__ int vt_pos(int k) {
  return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);
}

template <int D>
__global__ void __launch_bounds__(256)
v8_to_bf16_t_kernel(const int8_t* __restrict__ v, uint16_t* __restrict__ vt, int N, int Npad) {
  __shared__ int8_t tile[64][D + 4];
  const int64_t bh = blockIdx.y;
  const int n0 = blockIdx.x * 64;
  const int8_t* src = v + bh * (int64_t)N * D;
  for (int i = threadIdx.x; i < 64 * D / 16; i += 256) {
    const int r = i / (D / 16), c = (i % (D / 16)) * 16;
    uint4 x = {0, 0, 0, 0};
    if (n0 + r < N) x = *reinterpret_cast<const uint4*>(src + (int64_t)(n0 + r) * D + c);
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) *reinterpret_cast<uint32_t*>(&tile[r][c + 4 * e]) = w[e];
  }
  __syncthreads();
  uint16_t* dst = vt + bh * (int64_t)D * Npad + n0;
  for (int i = threadIdx.x; i < D * 32; i += 256) {
    const int d = i / 32, pr = (i % 32) * 2;  // storage positions pr, pr + 1
    const int k0 = (pr & ~15) + vt_pos(pr & 15);  // vt_pos is an involution; k0 + 1 pairs pr + 1
    const uint32_t lo = f2bf_bits((float)tile[k0][d]), hi = f2bf_bits((float)tile[k0 + 1][d]);
    *reinterpret_cast<uint32_t*>(dst + (int64_t)d * Npad + pr) = lo | (hi << 16);
  }
}

template <int VDT> struct PvOp;
template <> struct PvOp<SL8_DTYPE_F16> {
  typedef v8h vec;
  __device__ static vec pack(const float* p) {
    vec r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (_Float16)p[e];
    return r;
  }
  __device__ static v16f mfma(vec a, vec b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  // acc + sum of the 8 packed values (v_dot2_f32_f16 against ones): the row
  // sum of exactly the P that enters the PV product
  __device__ static float sum(vec v, const float*, float acc) {
    typedef _Float16 v2h __attribute__((ext_vector_type(2)));
    const v2h one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int e = 0; e < 8; e += 2) acc = __builtin_amdgcn_fdot2(v2h{v[e], v[e + 1]}, one, acc, false);
    return acc;
  }
  __device__ static void scale(vec& v, float s) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (_Float16)((float)v[e] * s);
  }
};
template <> struct PvOp<SL8_DTYPE_BF16> {
  typedef v8bf vec;
  __device__ static vec pack(const float* p) {
    vec r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (__bf16)p[e];
    return r;
  }
  __device__ static v16f mfma(vec a, vec b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // acc + sum of the 8 packed values (v_dot2_f32_bf16 against ones)
  __device__ static float sum(vec v, const float*, float acc) {
    typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
    const v2bf one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int e = 0; e < 8; e += 2)
      acc = __builtin_amdgcn_fdot2_f32_bf16(v2bf{v[e], v[e + 1]}, one, acc, false);
    return acc;
  }
  __device__ static void scale(vec& v, float s) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (__bf16)((float)v[e] * s);
  }
};

struct FwdArgs {
  const int8_t* q;
  const float* qs;
  const int8_t* k;
  const float* ks;
  const uint16_t* vt;  // V^T workspace
  void* out;
  float* lse;
  int32_t* scores;     // DUMP mode
  const float* vs;     // W8A8: per-channel V scale [B*Hkv][D]
  int M, N, Npad, Hq, Hkv, nqb, window_left;
  int diag;            // causal: query i sees keys <= i + diag
  int xcd_map;         // xcd_mode(): XCD-aware block order
  float w8_excess;     // W8A8: headroom of P above the reference point (log2)
  int dout;            // output row length (= D, or the caller's head dim when D is padded)
  const int32_t* skip; // production kernel: nonzero *skip -> every workgroup exits at once
};

// LDS tiles are dense; 16-byte chunks are XOR-swizzled within each row
// (chunk c of row r is stored at c ^ (r % chunks_per_row)) so that the
// MFMA operand reads of 8 consecutive rows hit distinct banks.

// blockIdx.x -> (b*Hq + h, query-block slot), heaviest slot first.
__device__ __forceinline__ void block_coords(const FwdArgs& a, int nslot, int& bh, int& slot) {
  attn_block_coords(a.Hq, a.Hkv, nslot, a.xcd_map, bh, slot);
}

template <int DC>
struct QOp {
  v4i c[DC];
};

// ---------------------------------------------------------------------------
// Production kernel. A wave owns NG x 32 queries (NG = 1: one MFMA column
// block) for the whole key loop; WV waves per workgroup (8 for D = 128, 4 for
// D = 64, halved down to 2 while the grid is smaller than the CU count; two
// waves per SIMD) share each 64-key K / k_scale / V^T tile, copied
// global -> LDS one tile ahead, so a larger workgroup means fewer copies per
// query. Each tile is processed as two 32-key half-steps; half-step h issues
// QK of half h and PV of half h-2 on the matrix cores while the VALU does the
// softmax of half h-1, so P stays in registers for one half-step. The
// reference point of the softmax is set once per row (see settle()) and O is
// never rescaled inside the loop.
// Per wave and tile (D = 128): 8 i8 + 16 f16 32x32 MFMAs, 24 KB of LDS
// operand reads (1 KB per MFMA), ~7 VALU operations per score.
// ---------------------------------------------------------------------------

#ifndef SL8_FWD_FAST
#define SL8_FWD_FAST 1
#endif
// operand prefetch distance of the straight-line half-steps (MFMAs ahead)
#ifndef SL8_FWD_PD
#define SL8_FWD_PD 3
#endif
#ifndef SL8_FWD_BAL
#define SL8_FWD_BAL 1
#endif
// balanced slices: the slot whose VALU slice starts the k_scale reads (config 2:
// slot 4 ~0.5 % faster than slot 6 on two machines)
#ifndef SL8_FWD_KVS
#define SL8_FWD_KVS 4
#endif
#ifndef SL8_FWD_OCC
#define SL8_FWD_OCC 2
#endif
// NG = 32-query MFMA column blocks per wave (1 or 2), WV = waves per
// workgroup (they share every K / V^T tile copied into LDS). W8 = the full
// W8A8 semantics (P re-quantised to int8 per 32-key half, int8 V with a
// per-channel scale); see half_probs_w8.
// DUMP = the same kernel with the int32 S^T tiles of every live 32-key half
// stored to a.scores [B*Hq][M][N] (the test hook that proves the production
// MFMA path's Q.K^T bit-exact); V and the scales are not read, nothing else
// is written.
template <int D, bool CAUSAL, int VDT, bool LSE, int NG, int WV, bool W8, bool DUMP = false>
__global__ void __launch_bounds__(WV * 64, (NG == 1 && D <= 128) ? SL8_FWD_OCC * 4 / WV : 1)
attn_fwd_wide_kernel(const FwdArgs a) {
  // the caller's accuracy gate fired: its result is discarded, so do nothing
  if (a.skip != nullptr && *a.skip != 0) return;
  constexpr int WT = WV * 64;                  // threads per workgroup
  // the straight-line steady-state half-step (half_step_fast): D = 128, NG = 1
  constexpr bool FAST = SL8_FWD_FAST && D == 128 && NG == 1 && !W8;
  // ... and its W8A8 counterpart (half_step_fast_w8): D = 256, NG = 1, lazy rescale
  constexpr bool FAST_W8 = SL8_FWD_FAST && D == 256 && NG == 1 && W8 && W8_LAZY;
  constexpr int WQ = 32 * NG;                  // queries per wave
  constexpr int WBM = WV * WQ;                 // queries per workgroup
  constexpr int DC = D / 32;
  constexpr int KCH = BN * D / 16 / WT;
  constexpr int VCH = D * BN * 2 / 16 / WT;
  static_assert(KCH >= 1 && VCH >= 1, "tile copies cover D in {64,128,256}");
  static_assert(!W8 || (VDT == SL8_DTYPE_BF16 && !LSE), "W8A8: bf16 PV, no LSE");
  static_assert(!DUMP || (!W8 && !LSE), "score dump: the int8 prefill only");
  __shared__ __attribute__((aligned(16))) int8_t sm_k0[BN * D];
  __shared__ __attribute__((aligned(16))) int8_t sm_k1[BN * D];
  __shared__ __attribute__((aligned(16))) uint16_t sm_v0[D * BN];
  __shared__ __attribute__((aligned(16))) uint16_t sm_v1[D * BN];
  __shared__ __attribute__((aligned(16))) float sm_s0[BN];
  __shared__ __attribute__((aligned(16))) float sm_s1[BN];
  using PV = PvOp<VDT>;
  typedef typename PV::vec pvec;

  const int nslot = CAUSAL ? (a.nqb + 1) / 2 : a.nqb;
  int bh, slot;
  block_coords(a, nslot, bh, slot);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  const int gsz = a.Hq / a.Hkv;
  const int b = bh / a.Hq, hq = bh % a.Hq;
  const int64_t bkv = (int64_t)b * a.Hkv + hq / gsz;
  const int M = a.M, N = a.N;
  const int diag = CAUSAL ? N - M : 0;
  const int wl = a.window_left;
  const int8_t* kb = a.k + bkv * (int64_t)N * D;
  const float* ksb = a.ks + bkv * (int64_t)N;
  // VT (the W8A8 variant): V^T [D][Npad] from v8_to_bf16_t_kernel; else V [N][D] in place
  constexpr bool VT = W8;
  const uint16_t* vb = a.vt + bkv * (int64_t)N * D;
  const uint16_t* vtb = a.vt + bkv * (int64_t)D * a.Npad;

  int qbs[2];
  int npass = 1;
  qbs[0] = a.nqb - 1 - slot;
  qbs[1] = slot;
  if (CAUSAL) npass = (qbs[1] != qbs[0]) ? 2 : 1;

  constexpr int KCPR = D / 16;
  // LDS has 64 four-byte banks (256 B): 16 lanes of a 16-byte read cover 16
  // consecutive tile rows, so a row's chunks are XOR-swizzled with the row's
  // index above the rows that share one 256-byte bank line (K rows: D bytes,
  // V^T rows: 128 bytes).
  constexpr int KSH = D == 256 ? 0 : (D == 128 ? 1 : 2);
  int koff[DC];
#pragma unroll
  for (int ch = 0; ch < DC; ++ch) koff[ch] = ((2 * ch + h) ^ ((l32 >> KSH) & (KCPR - 1))) * 16;
  // V tiles keep V's natural [key][D] layout in LDS; the PV A operand (32 dims
  // x 8 keys per lane) is read with ds_read_b64_tr_b16, which transposes 4 x 4
  // blocks of 16-bit values inside each 16-lane group (lane i, slot e <- lane
  // 4e + i/4, element i%4). Lane j of group G reads 4 dims of key row
  // kbase + 4h + j/4 (+8 for the second read): dims 32tt + 16(G%2) + 4(j%4).
  // Rows are XOR-swizzled in 64-byte units by (row & 3) (D = 64: by bit 1 of
  // the row; two rows share one 256-byte bank line) so the 32 lanes of a half
  // wave hit 32 distinct 8-byte bank slots. kbase + 4h is a multiple of 4, so
  // the swizzle is a per-lane constant.
  constexpr int VRB = 2 * D;  // bytes per V row
  const int vj = lane & 15, vrow = (vj >> 2) + 4 * h;
  const int vsw = D == 64 ? ((vj >> 3) & 1) : ((vj >> 2) & 3);
  int voffb[DC];
#pragma unroll
  for (int tt = 0; tt < DC; ++tt) {
    const int slot = 8 * tt + 4 * ((lane >> 4) & 1) + (vj & 3);  // 8-byte slot of the row
    voffb[tt] = vrow * VRB + 8 * (slot ^ (8 * vsw));
  }
  // VT: V^T tile [D][64 keys], rows of 128 bytes, 16-byte chunks swizzled by (row >> 1) & 7
  int voff[4];
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) voff[c4] = ((2 * c4 + h) ^ ((l32 >> 1) & 7)) * 8;
  // V buffers start as zeros (finite): the pipeline's first half-steps
  // multiply them by P = 0.
  for (int i = tid; i < D * BN / 8; i += WT) {
    reinterpret_cast<uint4*>(sm_v0)[i] = make_uint4(0, 0, 0, 0);
    reinterpret_cast<uint4*>(sm_v1)[i] = make_uint4(0, 0, 0, 0);
  }
  if constexpr (DUMP) {  // the scales are not read: unit k_scale keeps the softmax finite
    for (int i = tid; i < BN; i += WT) sm_s0[i] = sm_s1[i] = 1.f;
  }

  for (int pass = 0; pass < npass; ++pass) {
    const int m_blk = qbs[pass] * WBM;
    const int q0 = m_blk + wave * WQ;
    int mq[NG], qpos[NG];
    bool m_ok[NG];
    float qsc[NG];
    QOp<DC> qop[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      mq[g] = q0 + 32 * g + l32;
      m_ok[g] = mq[g] < M;
      qpos[g] = mq[g] + diag;
      const int8_t* qrow = a.q + ((int64_t)bh * M + (m_ok[g] ? mq[g] : M - 1)) * D + 16 * h;
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        qop[g].c[c] = *reinterpret_cast<const v4i*>(qrow + 32 * c);
        if (!m_ok[g]) qop[g].c[c] = v4i{0, 0, 0, 0};
      }
      qsc[g] = (m_ok[g] && !DUMP) ? a.qs[(int64_t)bh * M + mq[g]] : 1.f;
    }
    // seeded-accumulator constants of the straight-line path (see C0BITS)
    const float qs26 = qsc[0] * 67108864.f;  // q_scale * 2^26, exact
    const float cq26 = -(C0F * qs26);

    int n_end = N;
    if (CAUSAL) n_end = max(0, min(N, m_blk + WBM + diag));
    int n_beg = 0;
    if (wl >= 0) n_beg = min(n_end, max(0, m_blk + diag - wl + 1) & ~(BN - 1));
    const int ntiles = (n_end - n_beg + BN - 1) / BN;
    const int wq_lo = q0 + diag, wq_hi = q0 + WQ - 1 + diag;
    auto live = [&](int t) __attribute__((always_inline)) {
      if (t < 0 || t >= ntiles) return false;
      const int n0 = n_beg + t * BN;
      bool ok = true;
      if (CAUSAL && n0 > wq_hi) ok = false;
      if (wl >= 0 && n0 + BN - 1 <= wq_lo - wl) ok = false;
      return ok;
    };
    // the tile holds keys the wave must not see (bounds, causal, window)
    auto masked = [&](int t) __attribute__((always_inline)) {
      const int n0 = n_beg + t * BN;
      return (n0 + BN > N) || (CAUSAL && n0 + BN - 1 > wq_lo) || (wl >= 0 && n0 <= wq_hi - wl);
    };

    // Tile copies through buffer resources: per-lane byte offsets fixed for
    // the whole kernel, the tile start in the scalar offset; rows at or past N
    // read as zeros (their keys are masked).
    const brsrc_t rk = make_rsrc(kb, (uint32_t)N * D);
    const brsrc_t rv = VT ? make_rsrc(vtb, (uint32_t)D * a.Npad * 2) : make_rsrc(vb, (uint32_t)N * VRB);
    const brsrc_t rs = make_rsrc(ksb, (uint32_t)N * 4);
    uint32_t kvo[KCH], vvo[VCH];
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int sl = i * WT + tid;
      const int row = sl / KCPR;
      const int c = (sl % KCPR) ^ ((row >> KSH) & (KCPR - 1));
      kvo[i] = (uint32_t)(row * D + 16 * c);
    }
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int sl = i * WT + tid;
      if constexpr (VT) {
        const int row = sl / 8;
        const int c = (sl % 8) ^ ((row >> 1) & 7);
        vvo[i] = (uint32_t)(row * a.Npad * 2 + 16 * c);
      } else {
        // LDS chunk (row, c) holds V chunk c ^ 4k of key row n0 + row (k: the row's swizzle)
        const int row = sl / (D / 8);
        const int k = D == 64 ? ((row >> 1) & 1) : (row & 3);
        const int c = (sl % (D / 8)) ^ (4 * k);
        vvo[i] = (uint32_t)(row * VRB + 16 * c);
      }
    }
    auto load_k = [&](int n0, int8_t* dst) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < KCH; ++i)
        buf16_to_lds(rk, dst + (i * WT + wave * 64) * 16, kvo[i], (uint32_t)n0 * D);
    };
    auto load_v = [&](int n0, uint16_t* dst) __attribute__((always_inline)) {
      if constexpr (DUMP) return;
#pragma unroll
      for (int i = 0; i < VCH; ++i)
        buf16_to_lds(rv, dst + (i * WT + wave * 64) * 8, vvo[i], (uint32_t)n0 * (VT ? 2 : VRB));
    };
    auto load_s = [&](int n0, float* dst) __attribute__((always_inline)) {
      if constexpr (DUMP) return;
      if (wave == 0) buf4_to_lds(rs, dst, (uint32_t)lane * 4, (uint32_t)n0 * 4);
    };

    v16f oacc[NG][DC];
    float m_run[NG], l_lane[NG], mx_all[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) mx_all[g] = -INFINITY;
    bool ovf = false;
    bool all_set = false;  // every row's reference point is fixed (wave-uniform)

    // The key loop runs in half-steps of 32 keys (two per 64-key LDS tile).
    // Half-step h issues, as independent work for the matrix cores and VALU:
    //   QK of half h (MFMA)          scores of half h   (cvt, k_scale, mask, max)
    //   PV of half h-2 (MFMA)        P of half h-1      (exp2, pack, row sums)
    // then settles the reference point against the max of half h.
    typedef float xblk[NG][16];  // scaled scores of one half: [query block][key slot]
    typedef pvec pblk[NG][2];    // packed P of one half: [query block][16-key step]

    auto half_qk = [&](const int8_t* kt, int s, v16i (&sc)[NG]) __attribute__((always_inline)) {
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[g][r] = 0;
#pragma unroll
      for (int ch = 0; ch < DC; ++ch) {
        const v4i kop = *reinterpret_cast<const v4i*>(kt + (32 * s + l32) * D + koff[ch]);
#pragma unroll
        for (int g = 0; g < NG; ++g)
          sc[g] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kop, qop[g].c[ch], sc[g], 0, 0, 0);
      }
    };
    auto half_pv = [&](const uint16_t* vt, int s, const pblk& p) __attribute__((always_inline)) {
      typedef short v4s __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) v4s* lv4s_t;
      const char* vbytes = reinterpret_cast<const char*>(vt);
      if constexpr (VT) {
        const uint16_t* vr = vt + l32 * BN;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int tt = 0; tt < DC; ++tt) {
            const pvec vop = *reinterpret_cast<const pvec*>(vr + 32 * tt * BN + voff[2 * s + c]);
#pragma unroll
            for (int g = 0; g < NG; ++g) oacc[g][tt] = PV::mfma(vop, p[g][c], oacc[g][tt]);
          }
        return;
      }
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int tt = 0; tt < DC; ++tt) {
          const char* a0 = vbytes + (32 * s + 16 * c) * VRB + voffb[tt];
          const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lv4s_t)(a0));
          const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lv4s_t)(a0 + 8 * VRB));
          typedef short v8s __attribute__((ext_vector_type(8)));
          const v8s both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          const pvec vop = __builtin_bit_cast(pvec, both);
#pragma unroll
          for (int g = 0; g < NG; ++g) oacc[g][tt] = PV::mfma(vop, p[g][c], oacc[g][tt]);
        }
    };
    // t = acc * k_scale (logit = t * q_scale, q_scale > 0), masked; tile max
    auto half_scores = [&](const v16i (&sc)[NG], const float* st, int t, int s, bool do_mask,
                           bool dead, xblk& xo) __attribute__((always_inline)) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const float4 kv = *reinterpret_cast<const float4*>(st + 32 * s + 8 * gq + 4 * h);
        const float kk[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) xo[g][4 * gq + e] = (float)sc[g][4 * gq + e] * kk[e];
      }
      // Interleave the half-step's MFMAs (QK of this half, PV of half h-2)
      // with its LDS operand reads and VALU work (P of half h-1, the
      // conversion above), instead of issuing them as separate clusters.
      __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);  // LDS reads
#pragma unroll
      for (int i = 0; i < 3 * DC * NG; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, VT ? 1 : 2, 0);  // LDS reads
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
      }
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if (do_mask) {
          const int nb = n_beg + t * BN + 32 * s;
          // key n is visible iff n < N, n <= qpos (causal), n > qpos - wl
          // (window), i.e. (n - lo) unsigned < (hi - lo) with [lo, hi) the
          // visible range; one compare and one select per score
          const int hi = dead ? nb : min(N, CAUSAL ? qpos[g] + 1 : N);
          const int lo = (wl >= 0) ? qpos[g] - wl + 1 : INT_MIN / 2;
          const int lo_c = max(lo, nb - 64);
          const uint32_t span = hi > lo_c ? (uint32_t)(hi - lo_c) : 0u;
          const uint32_t rel = (uint32_t)(nb + 4 * h - lo_c);
          __builtin_amdgcn_sched_barrier(0);  // keep the mask compact (register pressure)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            xo[g][e] = (rel + (uint32_t)(8 * (e >> 2) + (e & 3)) < span) ? xo[g][e] : -INFINITY;
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    auto half_max = [&](const xblk& xo, float (&tmax)[NG]) __attribute__((always_inline)) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        float mx = -INFINITY;
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, xo[g][e]);
        tmax[g] = max_xor32(mx);
      }
    };
    // P = 2^(t*q_scale - m), packed per 16-key step, plus the row sums
    auto half_probs = [&](const xblk& xi, pblk& pc) __attribute__((always_inline)) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const float msub = (m_run[g] == -INFINITY) ? 0.f : m_run[g];
        float hs = 0.f;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          float pe[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) pe[e] = __builtin_amdgcn_exp2f(fmaf(xi[g][8 * c + e], qsc[g], -msub));
          pc[g][c] = PV::pack(pe);
          hs = PV::sum(pc[g][c], pe, hs);
        }
        l_lane[g] += hs;
        // some P above 2^15 (outside fp16) => the half's sum is too
        ovf = ovf || (hs > 32768.f);
      }
    };
    // Reference point (exp2 domain) per query: fixed by the first half that
    // has a visible key (O and l are still zero then, so nothing needs
    // rescaling) and never moved afterwards, so O is only ever touched by the
    // MFMAs inside the loop and no per-tile max is needed. P = 2^(logit -
    // m_ref) must stay within fp16; a half whose P sum exceeds 2^15 (implied
    // by any P > 2^15) sets ovf, and the pass is run again with m_ref = the
    // row max (found by a QK-only sweep).
    auto settle = [&](const xblk& xo) __attribute__((always_inline)) {
      bool unset = false;
#pragma unroll
      for (int g = 0; g < NG; ++g) unset = unset || (m_run[g] == -INFINITY);
      if (__any(unset)) {
        float tmax[NG];
        half_max(xo, tmax);
#pragma unroll
        for (int g = 0; g < NG; ++g)
          if (m_run[g] == -INFINITY) m_run[g] = tmax[g] * qsc[g];
      }
    };

    // W8A8 (reference attn_w8a8_fwd.cuh, per-warp quantisation): P of each
    // 32-key half is re-quantised against the half's own max,
    //   code = rint(127 * 2^(t - tmax_h)),
    // and enters the bf16 PV operand as code * 2^(tmax_h - m) / 127 (an
    // integer <= 127 times one per-row factor, applied before the product
    // instead of after the int32 sum). m is the row's reference point: set by
    // its first visible half (settle()) and moved up, with O and l rescaled,
    // only when a half's max exceeds it by more than a.w8_excess (~100 log2
    // units: bf16 P and the fp32 sums have the range), so rows with large
    // outliers rescale a few times instead of needing the exact row max from
    // a separate QK sweep (the W8_LAZY = false build: sweep, then one pass
    // with O never rescaled). The denominator sums the unquantised 2^(t - m).
    auto half_probs_w8 = [&](const xblk& xi, pblk& pc) __attribute__((always_inline)) {
      constexpr float LOG2_127 = 6.988684686772166f;
      float tm[NG];
      half_max(xi, tm);
#pragma unroll
      for (int g = 0; g < NG; ++g) tm[g] *= qsc[g];
      if constexpr (W8_LAZY) {
        // lazy rescale: a row whose half max exceeds its reference point by
        // more than a.w8_excess moves the point to that max, scaling its O
        // and l (O holds the products of halves up to h - 2, all relative to
        // the old point)
        const float excess = a.w8_excess;
        bool up = false;
#pragma unroll
        for (int g = 0; g < NG; ++g) up = up || (tm[g] > m_run[g] + excess);
        if (__any(up)) {
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            const bool ug = tm[g] > m_run[g] + excess;
            const float f = ug ? __builtin_amdgcn_exp2f(m_run[g] - tm[g]) : 1.f;
            if (ug) m_run[g] = tm[g];
            l_lane[g] *= f;
#pragma unroll
            for (int t = 0; t < DC; ++t)
#pragma unroll
              for (int r = 0; r < 16; ++r) oacc[g][t][r] *= f;
          }
        }
      }
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const bool any_key = tm[g] != -INFINITY;
        const float sub = any_key ? tm[g] - LOG2_127 : 0.f;
        const float fac = any_key ? __builtin_amdgcn_exp2f(tm[g] - m_run[g]) * (1.0f / 127.0f) : 0.f;
        float hs = 0.f;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          float pe[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float y = __builtin_amdgcn_exp2f(fmaf(xi[g][8 * c + e], qsc[g], -sub));
            hs += y;
            pe[e] = rintf(y) * fac;
          }
          pc[g][c] = PV::pack(pe);
        }
        l_lane[g] += hs * fac;
      }
    };

    // DUMP: the int32 scores of half s of tile t (keys n_beg + 64t + 32s ..),
    // stored where the tile is live for the wave; lane (h, l32) holds query
    // mq and keys 8(r / 4) + 4h + r % 4 of the half
    auto dump = [&](int g, const v16i& sc, int t, int s) __attribute__((always_inline)) {
      if constexpr (DUMP) {
        if (!live(t) || !m_ok[g]) return;
        int32_t* row = a.scores + ((int64_t)bh * M + mq[g]) * N;
        const int nb = n_beg + t * BN + 32 * s + 4 * h;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int n = nb + 8 * (r >> 2) + (r & 3);
          if (n < N) row[n] = sc[r];
        }
      }
    };

    xblk xA, xB;  // scores of the last two halves (alternating)
    pblk pA, pB;  // P of the last two halves (alternating)
    float xmA = -INFINITY, xmB = -INFINITY;  // W8A8 fast path: their row maxima (NG = 1)
    auto row_max = [&](const xblk& xo) __attribute__((always_inline)) {
      float t[NG];
      half_max(xo, t);
      return t[0];
    };
    // One half-step, a single straight-line block per variant: xi/p1 = the
    // half before (scores in, P out), xo = this half (scores out), p2 = P of
    // the half two back (consumed by PV). dead = this half has no tile (all
    // its scores -inf).
    auto half_step = [&](int j, int s, const int8_t* kt, const float* st, const uint16_t* vt,
                         bool mask, bool dead, xblk& xi, pblk& p1, xblk& xo,
                         pblk& p2) __attribute__((always_inline)) {
      v16i sc[NG];
      half_qk(kt, s, sc);
#pragma unroll
      for (int g = 0; g < NG; ++g) dump(g, sc[g], j, s);
      half_pv(vt, s, p2);
      half_probs(xi, p1);
      half_scores(sc, st, j, s, mask, dead, xo);
      settle(xo);
    };
    auto half_step_w8 = [&](int j, int s, const int8_t* kt, const float* st, const uint16_t* vt,
                            bool mask, bool dead, xblk& xi, pblk& p1, xblk& xo,
                            pblk& p2) __attribute__((always_inline)) {
      v16i sc[NG];
      half_qk(kt, s, sc);
      half_pv(vt, s, p2);
      half_probs_w8(xi, p1);
      half_scores(sc, st, j, s, mask, dead, xo);
      if constexpr (W8_LAZY) settle(xo);
    };
    // Steady-state half-step (no masked key, every row's reference point set):
    // one straight-line block in which MFMA i (QK of half h, then PV of half
    // h-2) is preceded by the LDS read of operand i + SL8_FWD_PD and followed by a
    // slice of the VALU work (P of half h-1, then the scores of half h), so
    // the matrix core never waits on an LDS round trip and the VALU runs
    // under the MFMAs. Same operations as half_step, in a fixed issue order.
    auto half_step_fast = [&](int j, int s, const int8_t* kt, const float* st, const uint16_t* vt,
                              xblk& xi, pblk& p1, xblk& xo, pblk& p2) __attribute__((always_inline)) {
      typedef short v4s __attribute__((ext_vector_type(4)));
      typedef short v8s __attribute__((ext_vector_type(8)));
      typedef __attribute__((address_space(3))) v4s* lv4s_t;
      if constexpr (FAST) {
      const char* vbytes = reinterpret_cast<const char*>(vt);
      // operand i of the half-step: i < DC: K chunk i (QK); else V^T (c, tt) for PV
      auto load_op = [&](int i) __attribute__((always_inline)) -> v4i {
        if (i < DC) return *reinterpret_cast<const v4i*>(kt + (32 * s + l32) * D + koff[i]);
        const int c = (i - DC) / DC, tt = (i - DC) % DC;
        const char* a0 = vbytes + (32 * s + 16 * c) * VRB + voffb[tt];
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lv4s_t)(a0));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lv4s_t)(a0 + 8 * VRB));
        const v8s both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        return __builtin_bit_cast(v4i, both);
      };
      constexpr int NOP = 3 * DC;
      const float msub = (m_run[0] == -INFINITY) ? 0.f : m_run[0];
      float pe[16];
      float hs = 0.f;
      float4 kv[4];
      v16i sc;
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[r] = C0BITS;
      v4i opb[NOP];  // operand i is read SL8_FWD_PD MFMAs ahead of its use
#pragma unroll
      for (int i = 0; i < SL8_FWD_PD && i < NOP; ++i) opb[i] = load_op(i);
      // Issue order, fixed by scheduling barriers: MFMA i is preceded by the
      // read of operand i + SL8_FWD_PD and followed by a slice of VALU work --
      //   QK MFMAs 0..3: P of half h-1, four exp2 each (xi holds the exp2 argument);
      //   PV MFMAs 0..1: pack P to fp16 + row sums (one 16-key step each);
      //   PV MFMA 2: k_scale reads; PV MFMAs 3..6: exp2 arguments of half h
      //   (two fmas each from the seeded accumulator, see C0BITS).
#pragma unroll
      for (int i = 0; i < NOP; ++i) {
        if (i + SL8_FWD_PD < NOP) opb[i + SL8_FWD_PD] = load_op(i + SL8_FWD_PD);
        __builtin_amdgcn_sched_barrier(0);  // the read goes out before MFMA i
        const v4i cur = opb[i];
#if SL8_FWD_BAL
        // Balanced slices (VALU cycles per MFMA slot ~32-40; exp2 is quarter
        // rate): slots 0..7 exp2 of keys 2i, 2i+1 of half h-1, with the pack +
        // row sum of keys 0..7 after slot 3 and of keys 8..15 after slot 7;
        // slot SL8_FWD_KVS reads k_scale, four slots before its first use;
        // slots 8..11 form the exp2 arguments of half h, four keys each (the QK
        // chain ended at slot 3).
        static_assert(NOP == 12, "balanced slices: D = 128");
        if (i < DC) sc = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur, qop[0].c[i], sc, 0, 0, 0);
        else oacc[0][(i - DC) % DC] = PV::mfma(__builtin_bit_cast(pvec, cur), p2[0][(i - DC) / DC],
                                               oacc[0][(i - DC) % DC]);
        if (i < 8) {
#pragma unroll
          for (int e = 2 * i; e < 2 * i + 2; ++e) {
            pe[e] = __builtin_amdgcn_exp2f(xi[0][e]);  // -inf -> 0
            pin_vgpr(pe[e]);
          }
        }
        if (i == 3 || i == 7) {
          const int k = i / 4;
          // same packing, row-sum order and overflow test as half_probs
          p1[0][k] = PV::pack(&pe[8 * k]);
          hs = PV::sum(p1[0][k], &pe[8 * k], hs);
          pin_vgpr(__builtin_bit_cast(v4i, p1[0][k]));
          pin_vgpr(hs);
          if (k == 1) {
            l_lane[0] += hs;
            ovf = ovf || (hs > 32768.f);
          }
        }
        if (i == SL8_FWD_KVS) {
#pragma unroll
          for (int gq = 0; gq < 4; ++gq)
            kv[gq] = *reinterpret_cast<const float4*>(st + 32 * s + 8 * gq + 4 * h);
        }
        if (i >= 8) {
          const int gq = i - 8;
          const float kk[4] = {kv[gq].x, kv[gq].y, kv[gq].z, kv[gq].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float w = fmaf(__int_as_float(sc[4 * gq + e]), qs26, cq26);
            xo[0][4 * gq + e] = fmaf(w, kk[e], -msub);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) pin_vgpr(xo[0][4 * gq + e]);
        }
#else
        if (i < DC) {
          sc = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur, qop[0].c[i], sc, 0, 0, 0);
#pragma unroll
          for (int e = 4 * i; e < 4 * i + 4; ++e) {
            pe[e] = __builtin_amdgcn_exp2f(xi[0][e]);  // -inf -> 0
            pin_vgpr(pe[e]);
          }
        } else {
          const int c = (i - DC) / DC, tt = (i - DC) % DC;
          oacc[0][tt] = PV::mfma(__builtin_bit_cast(pvec, cur), p2[0][c], oacc[0][tt]);
          const int k = i - DC;
          if (k < 2) {
            // same packing, row-sum order and overflow test as half_probs
            p1[0][k] = PV::pack(&pe[8 * k]);
            hs = PV::sum(p1[0][k], &pe[8 * k], hs);
            pin_vgpr(__builtin_bit_cast(v4i, p1[0][k]));
            pin_vgpr(hs);
            if (k == 1) {
              l_lane[0] += hs;
              ovf = ovf || (hs > 32768.f);
            }
          } else if (k == 2) {
#pragma unroll
            for (int gq = 0; gq < 4; ++gq)
              kv[gq] = *reinterpret_cast<const float4*>(st + 32 * s + 8 * gq + 4 * h);
          } else if (k < 7) {
            const int gq = k - 3;
            const float kk[4] = {kv[gq].x, kv[gq].y, kv[gq].z, kv[gq].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float w = fmaf(__int_as_float(sc[4 * gq + e]), qs26, cq26);
              xo[0][4 * gq + e] = fmaf(w, kk[e], -msub);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) pin_vgpr(xo[0][4 * gq + e]);
          }
        }
#endif
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (DUMP) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] -= C0BITS;  // the bits hold C0BITS + acc
        dump(0, sc, j, s);
      }
      }
    };

    // W8A8 steady-state half-step (D = 256, one wave per SIMD, so the schedule
    // inside the wave is all there is): the structure of half_step_fast with
    // half_probs_w8's arithmetic, including its lazy rescale (a branch taken
    // before the straight-line part, rarely).
    // xmi: the row max of xi (both lane halves), formed by the step that
    // produced xi (or by the fixup that changed it); this step forms xmo for
    // xo in the slices after its scores, so no max and no cross-lane round
    // trip stands between two half-steps.
    // pf: the first SL8_FWD_PD operands of half-step s, already read by the
    // step before it in the same tile (s = 1); step 0 reads them for step 1
    // in its last slices, so that no half-step inside a tile starts with a
    // full LDS round trip (one wave per SIMD: nothing else covers it).
    auto half_step_fast_w8 = [&](int s, const int8_t* kt, const float* st, const uint16_t* vt,
                                 xblk& xi, float xmi, pblk& p1, xblk& xo, float& xmo,
                                 pblk& p2, v4i (&pf)[SL8_FWD_PD]) __attribute__((always_inline)) {
      if constexpr (FAST_W8) {
      static_assert(SL8_FWD_PD <= DC, "the prefetched operands are K operands");
      constexpr float LOG2_127 = 6.988684686772166f;
      const uint16_t* vr = vt + l32 * BN;
      auto load_op = [&](int i) __attribute__((always_inline)) -> v4i {
        if (i < DC) return *reinterpret_cast<const v4i*>(kt + (32 * s + l32) * D + koff[i]);
        const int c = (i - DC) / DC, tt = (i - DC) % DC;
        return *reinterpret_cast<const v4i*>(vr + 32 * tt * BN + voff[2 * s + c]);
      };
      constexpr int NOP = 3 * DC;  // 8 QK + 16 PV MFMAs
      v4i opb[NOP];  // operand i is read SL8_FWD_PD MFMAs ahead of its use
      // the first operands go out before the reference-point arithmetic
#pragma unroll
      for (int i = 0; i < SL8_FWD_PD && i < NOP; ++i) opb[i] = s ? pf[i] : load_op(i);
      __builtin_amdgcn_sched_barrier(0);
      const float tm0 = xmi * qsc[0];
      // lazy rescale: the row's new reference point is used for this half's
      // codes now; O (which still gets half h-2's products, relative to the old
      // point, from the PV MFMAs below) and l are scaled after them
      const bool ug = tm0 > m_run[0] + a.w8_excess;
      const bool any_up = __any(ug);
      const float fr = ug ? __builtin_amdgcn_exp2f(m_run[0] - tm0) : 1.f;
      if (ug) m_run[0] = tm0;
      const bool any_key = tm0 != -INFINITY;
      const float sub = any_key ? tm0 - LOG2_127 : 0.f;
      const float fac = any_key ? __builtin_amdgcn_exp2f(tm0 - m_run[0]) * (1.0f / 127.0f) : 0.f;
      float pe[16];
      float hs = 0.f;
      float4 kv[4];
      float xm = -INFINITY;
      v16i sc;
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[r] = 0;
      // slices: QK MFMA i: P codes of keys 2i, 2i+1 of half h-1; PV MFMAs
      // 0..1: pack them (bf16) + row sum; PV 2: k_scale reads; PV 3..10:
      // scores of half h, two keys each; PV 11: their max in this lane;
      // PV 12: the max over both lane halves (xmo)
#pragma unroll
      for (int i = 0; i < NOP; ++i) {
        if (i + SL8_FWD_PD < NOP) opb[i + SL8_FWD_PD] = load_op(i + SL8_FWD_PD);
        __builtin_amdgcn_sched_barrier(0);  // the read goes out before MFMA i
        const v4i cur = opb[i];
        if (i < DC) {
          sc = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur, qop[0].c[i], sc, 0, 0, 0);
#pragma unroll
          for (int e = 2 * i; e < 2 * i + 2; ++e) {
            const float y = __builtin_amdgcn_exp2f(fmaf(xi[0][e], qsc[0], -sub));
            hs += y;
            pe[e] = rintf(y) * fac;
            pin_vgpr(pe[e]);
            pin_vgpr(hs);
          }
        } else {
          const int c = (i - DC) / DC, tt = (i - DC) % DC;
          oacc[0][tt] = PV::mfma(__builtin_bit_cast(pvec, cur), p2[0][c], oacc[0][tt]);
          const int k = i - DC;
          if (k < 2) {
            p1[0][k] = PV::pack(&pe[8 * k]);
            pin_vgpr(__builtin_bit_cast(v4i, p1[0][k]));
            if (k == 1) l_lane[0] = l_lane[0] * fr + hs * fac;
          } else if (k == 2) {
#pragma unroll
            for (int gq = 0; gq < 4; ++gq)
              kv[gq] = *reinterpret_cast<const float4*>(st + 32 * s + 8 * gq + 4 * h);
          } else if (k < 11) {
            const int e0 = 2 * (k - 3);
            const float ka[4] = {kv[e0 >> 2].x, kv[e0 >> 2].y, kv[e0 >> 2].z, kv[e0 >> 2].w};
            xo[0][e0] = (float)sc[e0] * ka[e0 & 3];
            xo[0][e0 + 1] = (float)sc[e0 + 1] * ka[(e0 + 1) & 3];
            pin_vgpr(xo[0][e0]);
            pin_vgpr(xo[0][e0 + 1]);
          } else if (k == 11) {
#pragma unroll
            for (int e = 0; e < 16; ++e) xm = fmaxf(xm, xo[0][e]);
            pin_vgpr(xm);
          } else if (k == 12) {
            xmo = max_xor32(xm);
            pin_vgpr(xmo);
          } else if (k >= 16 - SL8_FWD_PD && s == 0) {
            // the next half-step's first K operand (same tile, keys 32..63)
            const int n = k - (16 - SL8_FWD_PD);
            pf[n] = *reinterpret_cast<const v4i*>(kt + (32 + l32) * D + koff[n]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (any_up) {
#pragma unroll
        for (int t = 0; t < DC; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[0][t][r] *= fr;
      }
      }
    };

    // FAST path: xo already holds the exp2 argument logit - m (logit itself for a
    // row whose reference point is not set yet); a row set here shifts its xo
    auto settle_fast = [&](xblk& xo) __attribute__((always_inline)) {
      if (__any(m_run[0] == -INFINITY)) {
        float tmax[1];
        half_max(xo, tmax);
        if (m_run[0] == -INFINITY && tmax[0] != -INFINITY) {
          m_run[0] = tmax[0];
#pragma unroll
          for (int e = 0; e < 16; ++e) xo[0][e] -= tmax[0];
        }
      }
    };
    auto half_fixup = [&](int t, int s, bool do_mask, bool dead, xblk& xo) __attribute__((always_inline)) {
      if (do_mask) {
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          const int nb = n_beg + t * BN + 32 * s;
          // key n is visible iff (n - lo) unsigned < (hi - lo), [lo, hi) the visible range
          const int hi = dead ? nb : min(N, CAUSAL ? qpos[g] + 1 : N);
          const int lo = (wl >= 0) ? qpos[g] - wl + 1 : INT_MIN / 2;
          const int lo_c = max(lo, nb - 64);
          const uint32_t span = hi > lo_c ? (uint32_t)(hi - lo_c) : 0u;
          const uint32_t rel = (uint32_t)(nb + 4 * h - lo_c);
#pragma unroll
          for (int e = 0; e < 16; ++e)
            xo[g][e] = (rel + (uint32_t)(8 * (e >> 2) + (e & 3)) < span) ? xo[g][e] : -INFINITY;
        }
      }
      if constexpr (FAST) settle_fast(xo);
      else settle(xo);
      bool unset = false;
#pragma unroll
      for (int g = 0; g < NG; ++g) unset = unset || (m_run[g] == -INFINITY);
      all_set = !__any(unset);
    };

    // QK-only sweep: mx_all = the exact row max (exp2 domain) of the
    // visible logits, with the same double-buffered tile copies as the pass.
    auto sweep_tile = [&](int t, const int8_t* kc, const float* sc_, int8_t* kn, float* sn)
        __attribute__((always_inline)) {
      if (t + 1 < ntiles) {
        load_k(n_beg + (t + 1) * BN, kn);
        load_s(n_beg + (t + 1) * BN, sn);
      }
      if (live(t)) {
        const bool mk = masked(t);
        // both halves' MFMAs first: the second half's run under the first
        // half's conversion and max
        v16i sc0[NG], sc1[NG];
        xblk x0, x1;
        float t0[NG], t1[NG];
        half_qk(kc, 0, sc0);
        half_qk(kc, 1, sc1);
        half_scores(sc0, sc_, t, 0, mk, false, x0);
        half_max(x0, t0);
        half_scores(sc1, sc_, t, 1, mk, false, x1);
        half_max(x1, t1);
#pragma unroll
        for (int g = 0; g < NG; ++g) mx_all[g] = fmaxf(mx_all[g], fmaxf(t0[g], t1[g]) * qsc[g]);
      }
      wait_dma();
      __syncthreads();
    };
    auto sweep = [&]() __attribute__((always_inline)) {
      if (ntiles > 0) {
        load_k(n_beg, sm_k0);
        load_s(n_beg, sm_s0);
      }
      wait_dma();
      __syncthreads();
      int t = 0;
      for (; t + 1 < ntiles; t += 2) {
        sweep_tile(t, sm_k0, sm_s0, sm_k1, sm_s1);
        sweep_tile(t + 1, sm_k1, sm_s1, sm_k0, sm_s0);
      }
      if (t < ntiles) sweep_tile(t, sm_k0, sm_s0, sm_k1, sm_s1);
    };
    auto body = [&](int j, const int8_t* kcur, int8_t* knext, uint16_t* vcopy, const uint16_t* vprev,
                    const float* scur, float* snext) __attribute__((always_inline)) {
      const int n0 = n_beg + j * BN;
      auto copies_v = [&]() __attribute__((always_inline)) {
        if (j < ntiles) load_v(n0, vcopy);
      };
      auto copies_k = [&]() __attribute__((always_inline)) {
        if (j + 1 < ntiles) {
          load_k(n0 + BN, knext);
          load_s(n0 + BN, snext);
        }
      };
      auto copies = [&]() __attribute__((always_inline)) {
        if (j + 1 < ntiles) {
          load_k(n0 + BN, knext);
          load_s(n0 + BN, snext);
        }
        if (j < ntiles) load_v(n0, vcopy);
      };
      // The straight-line paths copy K and k_scale at the tile start and V
      // after the first half-step, so the two copies do not land in one burst
      // on top of a half-step's operand reads. Config 2: all copies after the
      // first half-step 126.4 us, split 124.9 us (V first, K after it: 125.9);
      // config 5: all at the start 1100 us, all after the first half-step
      // 1128 us, split 1082 us (V first, K after it: 1135 us).
      if constexpr (!FAST && !FAST_W8) copies();
      if constexpr (FAST || FAST_W8) copies_k();
      const bool dead = !live(j);
      const bool mask = dead || masked(j);
      // A dead tile after a dead tile has nothing to do: the one before already
      // pushed the last visible half's P through PV, and what it left pending
      // is P = 0 and scores of -inf (in the diagonal block, the waves whose
      // queries end early skip their last tiles this way).
      if (dead && !live(j - 1)) {
        if constexpr (FAST || FAST_W8) copies_v();
      } else if constexpr (W8) {
        if constexpr (FAST_W8) {
          // a fixup may mask scores: the carried max is formed again
          v4i pf[SL8_FWD_PD];
          half_step_fast_w8(0, kcur, scur, vprev, xB, xmB, pB, xA, xmA, pA, pf);
          if (mask || !all_set) {
            half_fixup(j, 0, mask, dead, xA);
            xmA = row_max(xA);
          }
          copies_v();
          half_step_fast_w8(1, kcur, scur, vprev, xA, xmA, pA, xB, xmB, pB, pf);
          if (mask || !all_set) {
            half_fixup(j, 1, mask, dead, xB);
            xmB = row_max(xB);
          }
        } else {
          half_step_w8(j, 0, kcur, scur, vprev, mask, dead, xB, pB, xA, pA);
          half_step_w8(j, 1, kcur, scur, vprev, mask, dead, xA, pA, xB, pB);
        }
      } else {
        if constexpr (FAST) {
          // a masked half, or one that may fix some row's reference point,
          // gets its mask / settle after the straight-line part
          half_step_fast(j, 0, kcur, scur, vprev, xB, pB, xA, pA);
          if (mask || !all_set) half_fixup(j, 0, mask, dead, xA);
          copies_v();
          half_step_fast(j, 1, kcur, scur, vprev, xA, pA, xB, pB);
          if (mask || !all_set) half_fixup(j, 1, mask, dead, xB);
        } else {
          half_step(j, 0, kcur, scur, vprev, mask, dead, xB, pB, xA, pA);
          half_step(j, 1, kcur, scur, vprev, mask, dead, xA, pA, xB, pB);
          bool unset = false;
#pragma unroll
          for (int g = 0; g < NG; ++g) unset = unset || (m_run[g] == -INFINITY);
          all_set = !__any(unset);
        }
      }
      wait_dma();
      __syncthreads();
    };
    if constexpr (W8 && !W8_LAZY) sweep();
    for (int attempt = (W8 && !W8_LAZY) ? 1 : 0; attempt < 2; ++attempt) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
#pragma unroll
        for (int t = 0; t < DC; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[g][t][r] = 0.f;
        // second run: the row max of the first one, which no logit exceeds
        m_run[g] = attempt ? mx_all[g] : -INFINITY;
        l_lane[g] = 0.f;
      }
      ovf = false;
      all_set = false;
      // Iteration j reads K_j, k_scale_j (halves 2j, 2j+1) and V_{j-1} (PV of
      // halves 2j-2, 2j-1), and copies K_{j+1}, k_scale_{j+1} and V_j into the
      // other buffers.
      if (ntiles > 0) {
        load_k(n_beg, sm_k0);
        load_s(n_beg, sm_s0);
      }
      wait_dma();
      __syncthreads();

      // Pipeline state before the first half: scores -inf (P = 0) and P = 0, so
      // the first two half-steps add nothing; the V buffers are zeroed once so
      // those products are 0 * finite.
  #pragma unroll
      for (int g = 0; g < NG; ++g) {
  #pragma unroll
        for (int e = 0; e < 16; ++e) xA[g][e] = xB[g][e] = -INFINITY;
        xmA = xmB = -INFINITY;
  #pragma unroll
        for (int c = 0; c < 2; ++c) {
          float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
          pA[g][c] = PV::pack(z);
          pB[g][c] = pA[g][c];
        }
      }
      // both bodies unconditional inside the loop (keeps every accumulator
      // update in place); an odd last iteration is peeled
      int j = 0;
      for (; j + 1 <= ntiles; j += 2) {
        body(j, sm_k0, sm_k1, sm_v0, sm_v1, sm_s0, sm_s1);
        body(j + 1, sm_k1, sm_k0, sm_v1, sm_v0, sm_s1, sm_s0);
      }
      if (j <= ntiles) body(j, sm_k0, sm_k1, sm_v0, sm_v1, sm_s0, sm_s1);

      if (DUMP || !__syncthreads_or(ovf ? 1 : 0)) break;
      // QK-only sweep for the exact row max (the whole workgroup takes part)
      sweep();
    }

#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if constexpr (DUMP) break;
      const float l = l_lane[g] + __shfl_xor(l_lane[g], 32, 64);
      if (m_ok[g]) {
        const float inv = (l > 0.f) ? 1.f / l : 0.f;
        uint16_t* orow = reinterpret_cast<uint16_t*>(a.out) + ((int64_t)bh * M + mq[g]) * a.dout;
#pragma unroll
        for (int tt = 0; tt < DC; ++tt)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            if (32 * tt + 8 * gq + 4 * h >= a.dout) continue;  // zero-padded channels
            float vsc[4] = {1.f, 1.f, 1.f, 1.f};
            if constexpr (W8) {
              const float4 v4 = *reinterpret_cast<const float4*>(a.vs + bkv * D + 32 * tt + 8 * gq + 4 * h);
              vsc[0] = v4.x; vsc[1] = v4.y; vsc[2] = v4.z; vsc[3] = v4.w;
            }
            uint16_t hv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float xo = oacc[g][tt][4 * gq + e] * inv * vsc[e];
              hv[e] = (W8 || VDT == SL8_DTYPE_F16) ? f2h_bits(xo) : f2bf_bits(xo);  // W8A8 out: fp16
            }
            uint2 pk;
            pk.x = hv[0] | ((uint32_t)hv[1] << 16);
            pk.y = hv[2] | ((uint32_t)hv[3] << 16);
            *reinterpret_cast<uint2*>(orow + 32 * tt + 8 * gq + 4 * h) = pk;
          }
        if (LSE && h == 0)
          a.lse[(int64_t)bh * M + mq[g]] = (l > 0.f) ? (m_run[g] * LN2F + logf(l)) : -INFINITY;
      }
    }
  }
}

// query-column blocks per wave of the production kernel
#ifndef SL8_FWD_NG
#define SL8_FWD_NG 1
#endif
constexpr int WIDE_NG = SL8_FWD_NG;
// waves per workgroup of the production kernel, per head dim
#ifndef SL8_FWD_WV128
#define SL8_FWD_WV128 8
#endif
#ifndef SL8_FWD_WV64
#define SL8_FWD_WV64 4
#endif
// (D = 256 keeps 4: one wave per SIMD, whose O needs the whole register file)
constexpr int wide_waves(int64_t D) { return D == 128 ? SL8_FWD_WV128 : (D == 64 ? SL8_FWD_WV64 : 4); }
// queries per workgroup
#ifndef SL8_FWD_NG256
#define SL8_FWD_NG256 1
#endif
constexpr int wide_ng(int64_t D) { return D == 256 ? SL8_FWD_NG256 : WIDE_NG; }
constexpr int wide_bm(int64_t D) { return wide_waves(D) * 32 * wide_ng(D); }

template <int D, bool CAUSAL, int VDT, bool LSE, bool W8 = false, int WV = wide_waves(D)>
void launch_wide(const FwdArgs& a, int grid, hipStream_t st) {
  attn_fwd_wide_kernel<D, CAUSAL, VDT, LSE, wide_ng(D), WV, W8><<<grid, WV * 64, 0, st>>>(a);
}

// Small grids (short sequences, few heads): fewer waves per workgroup, i.e.
// fewer queries per workgroup and more workgroups, until the grid covers the
// CUs (the waves per SIMD stay 2: see the launch bounds). D = 128: 8, 4 or 2
// waves; D = 64: 4 or 2; D = 256 keeps 4.
#ifndef SL8_FWD_SMALLGRID
#define SL8_FWD_SMALLGRID 1
#endif
int wide_waves_for(int64_t DP, int64_t B, int64_t Hq, int64_t M, bool causal) {
  int wv = wide_waves(DP);
  if (!SL8_FWD_SMALLGRID || (DP != 128 && DP != 64) || wide_ng(DP) != 1) return wv;
  const int64_t cus = cu_count();
  while (wv > 2) {
    const int64_t bm = (int64_t)wv * 32, nqb = (M + bm - 1) / bm;
    const int64_t grid = B * Hq * (causal ? (nqb + 1) / 2 : nqb);
    if (grid >= cus) break;
    wv /= 2;
  }
  return wv;
}

template <int D, int VDT, int WV>
void dispatch_wide_wv(const FwdArgs& a, int grid, bool causal, bool lse, hipStream_t st) {
  if (causal) {
    if (lse) launch_wide<D, true, VDT, true, false, WV>(a, grid, st);
    else launch_wide<D, true, VDT, false, false, WV>(a, grid, st);
  } else {
    if (lse) launch_wide<D, false, VDT, true, false, WV>(a, grid, st);
    else launch_wide<D, false, VDT, false, false, WV>(a, grid, st);
  }
}

template <int D, int VDT>
void dispatch_wide(const FwdArgs& a, int grid, bool causal, bool lse, int wv, hipStream_t st) {
  if constexpr (D == 128) {
    if (wv == 2) return dispatch_wide_wv<D, VDT, 2>(a, grid, causal, lse, st);
    if (wv == 4) return dispatch_wide_wv<D, VDT, 4>(a, grid, causal, lse, st);
  } else if constexpr (D == 64) {
    if (wv == 2) return dispatch_wide_wv<D, VDT, 2>(a, grid, causal, lse, st);
  }
  dispatch_wide_wv<D, VDT, wide_waves(D)>(a, grid, causal, lse, st);
}

int64_t npad_of(int64_t N) { return (N + BN - 1) / BN * BN; }


int check_fwd_shape(int64_t B, int64_t Hq, int64_t Hkv, int64_t M, int64_t N, int64_t D) {
  SL8_CHECK_ARG(B >= 0 && Hq >= 0 && Hkv > 0 && M >= 0 && N >= 0, "fni8: bad shape");
  SL8_CHECK_ARG(Hq % Hkv == 0, "fni8: H_q must be divisible by H_kv (GQA)");
  SL8_CHECK_ARG(D == 32 || D == 64 || D == 72 || D == 80 || D == 128 || D == 256,
                "fni8: head dim must be 32/64/72/80/128/256, got %lld", (long long)D);
  SL8_CHECK_ARG(M < (1 << 30) && N < (1 << 30) && B * Hq < (1 << 24), "fni8: shape too large");
  // one KV head's V (and W8A8's padded V^T) is addressed by a 32-bit buffer offset
  SL8_CHECK_ARG(N * 2 * (D + 64) < (1LL << 31), "fni8: shape too large (N=%lld)", (long long)N);
  return SL8_OK;
}

// launch geometry of the production kernel for (padded) head dim DP: query
// blocks of wv x 32 x wide_ng(DP) rows (wv = 0: wide_waves(DP)); causal launches pair block qb with nqb-1-qb, so
// the grid holds (nqb + 1) / 2 slots per head
FwdArgs make_args(int64_t B, int64_t Hq, int64_t Hkv, int64_t M, int64_t N, int64_t DP,
                  bool causal, int& grid, int wv = 0) {
  const int bm = (wv > 0 ? wv : wide_waves(DP)) * 32 * wide_ng(DP);
  FwdArgs a{};
  a.M = (int)M;
  a.N = (int)N;
  a.Npad = (int)npad_of(N);
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.nqb = (int)((M + bm - 1) / bm);
  a.window_left = -1;
  a.diag = (int)(N - M);
  a.dout = 0;  // set by the callers
  const int nslot = causal ? (a.nqb + 1) / 2 : a.nqb;
  grid = (int)(B * Hq * nslot);
  a.xcd_map = xcd_mode(B * Hkv, Hq / Hkv, nslot);
  return a;
}

}  // namespace

namespace {

// ---------------------------------------------------------------------------
// Head dims without an MFMA tiling of their own (32, 72, 80) run on the
// kernel of the next supported width DP (64 or 128): Q, K and V rows are
// copied into a workspace zero-padded to DP channels. Zero channels add
// nothing to the int32 Q.K^T sums (the scores are bit-identical) and give
// zero output channels, which the epilogue does not store (FwdArgs::dout).
// ---------------------------------------------------------------------------
int padded_head_dim(int64_t D) { return D == 32 ? 64 : (D == 72 || D == 80) ? 128 : (int)D; }

// dst[r][0 .. dw) = src[r][0 .. sw) followed by zeros, in dwords
__global__ void __launch_bounds__(256)
pad_rows_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, int64_t rows, int sw,
                int dw) {
  const int64_t total = rows * dw;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / dw;
    const int c = (int)(i - r * dw);
    dst[i] = c < sw ? src[r * sw + c] : 0u;
  }
}

// row bytes must be multiples of 4 (every head dim here is a multiple of 8)
int pad_rows(const void* src, void* dst, int64_t rows, int64_t src_bytes, int64_t dst_bytes,
             hipStream_t st) {
  if (rows <= 0) return SL8_OK;
  const int64_t total = rows * (dst_bytes / 4);
  const int64_t grid = std::min<int64_t>((total + 255) / 256, 8192);
  pad_rows_kernel<<<(unsigned)grid, 256, 0, st>>>(static_cast<const uint32_t*>(src),
                                                   static_cast<uint32_t*>(dst), rows,
                                                   (int)(src_bytes / 4), (int)(dst_bytes / 4));
  SL8_CHECK_LAUNCH("pad head dim");
  return SL8_OK;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// workspace of the padded operands: Q [B*Hq*M][DP], K [B*Hkv*N][DP] (int8),
// V [B*Hkv*N][DP] of v_bytes per element, and (W8A8) v_scale [B*Hkv][DP]
size_t pad_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t M, int64_t N, int64_t D,
                     int v_bytes, bool vscale) {
  const int64_t DP = padded_head_dim(D);
  if (DP == D || B <= 0) return 0;
  return align256((size_t)(B * Hq * M * DP)) + align256((size_t)(B * Hkv * N * DP)) +
         align256((size_t)(B * Hkv * N * DP * v_bytes)) +
         (vscale ? align256((size_t)(B * Hkv * DP * 4)) : 0);
}

struct Padded {
  const int8_t* q;
  const int8_t* k;
  const void* v;
  const float* vs;
  void* rest;  // workspace past the padded operands
};

int pad_operands(const int8_t* q, const int8_t* k, const void* v, const float* vs, int64_t B,
                 int64_t Hq, int64_t Hkv, int64_t M, int64_t N, int64_t D, int v_bytes, void* ws,
                 hipStream_t st, Padded& p) {
  const int64_t DP = padded_head_dim(D);
  char* w = static_cast<char*>(ws);
  char* qp = w;
  w += align256((size_t)(B * Hq * M * DP));
  char* kp = w;
  w += align256((size_t)(B * Hkv * N * DP));
  char* vp = w;
  w += align256((size_t)(B * Hkv * N * DP * v_bytes));
  char* vsp = w;
  int rc = pad_rows(q, qp, B * Hq * M, D, DP, st);
  if (!rc) rc = pad_rows(k, kp, B * Hkv * N, D, DP, st);
  if (!rc && v) rc = pad_rows(v, vp, B * Hkv * N, D * v_bytes, DP * v_bytes, st);
  if (!rc && vs) {
    rc = pad_rows(vs, vsp, B * Hkv, D * 4, DP * 4, st);
    w += align256((size_t)(B * Hkv * DP * 4));
  }
  p = Padded{reinterpret_cast<int8_t*>(qp), reinterpret_cast<int8_t*>(kp), vp,
             vs ? reinterpret_cast<float*>(vsp) : nullptr, w};
  return rc;
}

}  // namespace

// largest P exponent that keeps the W8A8 sums of N keys below 2^120
float w8_excess_for(int64_t N) {
  int lg = 0;
  while (lg < 62 && (1LL << lg) < N) ++lg;
  return (float)std::max(16, 120 - 7 - lg);
}

size_t w8a8_wide_workspace(int64_t B, int64_t Hkv, int64_t N, int64_t D) {
  return (size_t)(B * Hkv * padded_head_dim(D) * npad_of(N)) * sizeof(uint16_t);
}

// padded operands (int8 Q/K/V and the per-channel V scale) of a W8A8 call
size_t w8a8_pad_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t M, int64_t N, int64_t D) {
  return pad_workspace(B, Hq, Hkv, M, N, D, 1, true);
}

int w8a8_pad_operands(const int8_t*& q, const int8_t*& k, const int8_t*& v, const float*& vs,
                      int64_t B, int64_t Hq, int64_t Hkv, int64_t M, int64_t N, int64_t D,
                      void*& ws, hipStream_t st) {
  if (padded_head_dim(D) == D) return SL8_OK;
  Padded p;
  const int rc = pad_operands(q, k, v, vs, B, Hq, Hkv, M, N, D, 1, ws, st, p);
  q = p.q;
  k = p.k;
  v = static_cast<const int8_t*>(p.v);
  vs = p.vs;
  ws = p.rest;
  return rc;
}

// W8A8 prefill with per-warp P quantisation on the production pipeline
// (called from attn_w8a8.hip). v: int8 [B*Hkv][N][D]; vt_ws: workspace of
// w8a8_wide_workspace() bytes for bf16 V^T [B*Hkv][D][Npad]. D is a
// supported width (64/128/256); dout = the output row length (the caller's
// head dim when the operands were padded).
// ---------------------------------------------------------------------------
// W8A8 prefill at D = 256 with 16 queries per wave (SL8_W8_Q16). The 32-query
// waves of attn_fwd_wide_kernel hold O in 128 accumulators and run one wave
// per SIMD, where nothing covers a wave's own latencies or the per-tile
// barrier. Here a wave owns 16 queries on the 16x16 MFMAs: O^T is 16 blocks
// of 16 dims x 16 queries (64 accumulators), and a workgroup of 8 waves (two
// per SIMD) covers the same 128 queries and shares the same K / V^T tiles.
//   QK: S^T = K Q^T on v_mfma_i32_16x16x64_i8, per 32-key half 2 key blocks
//       x 4 dim chunks. A-operand row r of a block is key rho(r) =
//       8 ((r / 4) & 1) + 4 (r / 8) + r % 4 (any row order is valid), so lane
//       (l16, g) ends with keys 16 kb + kg + i of query l16, kg = rho(4 g)
//       (kb = 0, 1; i = 0..3).
//   PV: O^T += V^T P^T on v_mfma_f32_16x16x32_bf16 with the half's 32 keys in
//       the order sigma(8 g + e) = 16 (e / 4) + kg + e % 4: exactly the keys
//       lane (l16, g) holds, so P needs no lane exchange; the V^T operand is
//       two 8-byte reads per MFMA in the same order. rho makes lane groups
//       g = 0, 1 (one pass of an 8-byte LDS read) read the two 8-byte halves
//       of their chunks: with keys 4 g + i they read the same half and
//       collided 2-way on every V^T read (LDS bank conflicts ~23 % of the
//       launch at config 5).
// The arithmetic per row is the wide kernel's W8A8 path (P re-quantised per
// 32-key half against the half's max, the lazy reference-point rescale), and
// so is the straight-line half-step. Config 5: 1081 -> 986 us (the same
// kernel with the compiler's schedule, each operand read right before its
// MFMA: 1633 us). SL8_W8_Q16 = 0 runs attn_fwd_wide_kernel's W8A8 path.
#ifndef SL8_W8_Q16
#define SL8_W8_Q16 1
#endif
#ifndef SL8_Q16_PD
#define SL8_Q16_PD 4  // operand reads ahead of their MFMA (2 / 3 / 4 / 6 at config 5: 972 / 969 / 963 / 967 us)
#endif
typedef float v4f_t __attribute__((ext_vector_type(4)));

namespace {

template <bool CAUSAL>
__global__ void __launch_bounds__(512, 1)
attn_w8a8_q16_kernel(const FwdArgs a) {
  if (a.skip != nullptr && *a.skip != 0) return;
  constexpr int D = 256, WT = 512, WQ = 16, WBM = 128;
  constexpr int KCH = BN * D / 16 / WT;      // K tile copies per thread
  constexpr int VCH = D * BN * 2 / 16 / WT;  // V^T tile copies per thread
  constexpr float LOG2_127 = 6.988684686772166f;
  __shared__ __attribute__((aligned(16))) int8_t sk0[BN * D];
  __shared__ __attribute__((aligned(16))) int8_t sk1[BN * D];
  __shared__ __attribute__((aligned(16))) uint16_t sv0[D * BN];
  __shared__ __attribute__((aligned(16))) uint16_t sv1[D * BN];
  __shared__ __attribute__((aligned(16))) float ss0[BN];
  __shared__ __attribute__((aligned(16))) float ss1[BN];

  const int nslot = CAUSAL ? (a.nqb + 1) / 2 : a.nqb;
  int bh, slot;
  block_coords(a, nslot, bh, slot);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int gsz = a.Hq / a.Hkv;
  const int b = bh / a.Hq, hq = bh % a.Hq;
  const int64_t bkv = (int64_t)b * a.Hkv + hq / gsz;
  const int M = a.M, N = a.N;
  const int diag = CAUSAL ? N - M : 0;
  const int wl = a.window_left;
  const int8_t* kb = a.k + bkv * (int64_t)N * D;
  const float* ksb = a.ks + bkv * (int64_t)N;
  const uint16_t* vtb = a.vt + bkv * (int64_t)D * a.Npad;

  int qbs[2];
  int npass = 1;
  qbs[0] = a.nqb - 1 - slot;
  qbs[1] = slot;
  if (CAUSAL) npass = (qbs[1] != qbs[0]) ? 2 : 1;

  // K operand (A, 16 keys x 64 dims): lane (l16, g) reads the 16-byte chunk
  // 4 c + g of key row l16 of the block; the tile keeps chunk c of row r at
  // c ^ (r & 15) (the copy below), so 16 rows read 16 distinct bank groups
  const int rl = 8 * ((l16 >> 2) & 1) + 4 * (l16 >> 3) + (l16 & 3);  // rho(l16)
  const int kg = 8 * (g & 1) + 4 * (g >> 1);                          // rho(4 g)
  int koff[4];
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) koff[c4] = ((4 * c4 + g) ^ rl) * 16;
  // V^T operand (A, 16 dims x 32 keys in sigma order): keys kg .. +3 and
  // 16 + kg .. +3 of the half, 8 bytes each, of V^T row l16 of the dim
  // block. v8_to_bf16_t_kernel stores each 16-key group with bits 2 and 3 of
  // the key index exchanged (key 8 b3 + 4 b2 + i at position 8 b2 + 4 b3 + i),
  // so keys kg + i = 8 (g & 1) + 4 (g >> 1) + i of a group sit at
  // 8 (g >> 1) + 4 (g & 1) + i: chunk (g >> 1) of the group, byte 8 (g & 1);
  // the tile keeps 16-byte chunk c of row d at c ^ ((d >> 1) & 7)
  int voff[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int p = 0; p < 2; ++p)
      voff[s][p] = ((4 * s + 2 * p + (g >> 1)) ^ ((l16 >> 1) & 7)) * 16 + (g & 1) * 8;
  // V buffers start as zeros (finite): the first half-steps multiply them by P = 0
  for (int i = tid; i < D * BN / 8; i += WT) {
    reinterpret_cast<uint4*>(sv0)[i] = make_uint4(0, 0, 0, 0);
    reinterpret_cast<uint4*>(sv1)[i] = make_uint4(0, 0, 0, 0);
  }

  for (int pass = 0; pass < npass; ++pass) {
    const int m_blk = qbs[pass] * WBM;
    const int q0 = m_blk + wave * WQ;
    const int mq = q0 + l16;
    const bool m_ok = mq < M;
    const int qpos = mq + diag;
    // Q operand (B, 64 dims x 16 queries): query mq, dims 64 c + 16 g .. +15
    v4i qop[4];
    {
      const int8_t* qrow = a.q + ((int64_t)bh * M + (m_ok ? mq : M - 1)) * D + 16 * g;
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        qop[c4] = *reinterpret_cast<const v4i*>(qrow + 64 * c4);
        if (!m_ok) qop[c4] = v4i{0, 0, 0, 0};
      }
    }
    const float qsc = m_ok ? a.qs[(int64_t)bh * M + mq] : 1.f;

    int n_end = N;
    if (CAUSAL) n_end = max(0, min(N, m_blk + WBM + diag));
    int n_beg = 0;
    if (wl >= 0) n_beg = min(n_end, max(0, m_blk + diag - wl + 1) & ~(BN - 1));
    const int ntiles = (n_end - n_beg + BN - 1) / BN;
    const int wq_lo = q0 + diag, wq_hi = q0 + WQ - 1 + diag;
    auto live = [&](int t) __attribute__((always_inline)) {
      if (t < 0 || t >= ntiles) return false;
      const int n0 = n_beg + t * BN;
      bool ok = true;
      if (CAUSAL && n0 > wq_hi) ok = false;
      if (wl >= 0 && n0 + BN - 1 <= wq_lo - wl) ok = false;
      return ok;
    };
    auto masked = [&](int t) __attribute__((always_inline)) {
      const int n0 = n_beg + t * BN;
      return (n0 + BN > N) || (CAUSAL && n0 + BN - 1 > wq_lo) || (wl >= 0 && n0 <= wq_hi - wl);
    };

    // tile copies, as the wide kernel's (rows past N read as zeros)
    const brsrc_t rk = make_rsrc(kb, (uint32_t)N * D);
    const brsrc_t rv = make_rsrc(vtb, (uint32_t)D * a.Npad * 2);
    const brsrc_t rs = make_rsrc(ksb, (uint32_t)N * 4);
    uint32_t kvo[KCH], vvo[VCH];
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int sl = i * WT + tid;
      const int row = sl / 16;
      const int c = (sl % 16) ^ (row & 15);
      kvo[i] = (uint32_t)(row * D + 16 * c);
    }
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int sl = i * WT + tid;
      const int row = sl / 8;
      const int c = (sl % 8) ^ ((row >> 1) & 7);
      vvo[i] = (uint32_t)(row * a.Npad * 2 + 16 * c);
    }
    auto load_k = [&](int n0, int8_t* dst) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < KCH; ++i)
        buf16_to_lds(rk, dst + (i * WT + wave * 64) * 16, kvo[i], (uint32_t)n0 * D);
    };
    auto load_v = [&](int n0, uint16_t* dst) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < VCH; ++i)
        buf16_to_lds(rv, dst + (i * WT + wave * 64) * 8, vvo[i], (uint32_t)n0 * 2);
    };
    auto load_s = [&](int n0, float* dst) __attribute__((always_inline)) {
      if (wave == 0) buf4_to_lds(rs, dst, (uint32_t)lane * 4, (uint32_t)n0 * 4);
    };

    v4f_t oacc[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) oacc[t] = v4f_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_lane = 0.f;
    typedef float xblk16[8];  // a half's scores: slot 4 kb + i = key 16 kb + kg + i

    // max over the 32 keys of the row: the lane's 8, then the 4 lane groups
    auto row_max = [&](const xblk16& x) __attribute__((always_inline)) {
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, x[e]);
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
      return max_xor32(mx);
    };
    xblk16 xA, xB;
    v8bf pA, pB;
    float xmA = -INFINITY, xmB = -INFINITY;  // their row maxima (both lane groups)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xA[e] = xB[e] = -INFINITY;
      pA[e] = pB[e] = (__bf16)0.f;
    }
    bool all_set = false;  // every row's reference point is fixed (wave-uniform)
    // Straight-line half-step (the wide kernel's half_step_fast_w8 in this
    // layout): MFMA i (QK of half h: i < 8; PV of half h - 2: i >= 8) is
    // preceded by the LDS read of operand i + 3 and followed by a slice of
    // VALU work: P code of key i of half h - 1 (i < 8); the k_scale reads and
    // the pack of P (i = 8); the score of key i - 9 of half h (i = 9..16);
    // its max (i = 17, 18). xmi: the row max of xi; xmo: that of xo (before
    // masking: the fixup forms it again).
    auto half_step_fast = [&](int s, const int8_t* kt, const float* st, const uint16_t* vt,
                              xblk16& xi, float xmi, v8bf& p1, xblk16& xo, float& xmo,
                              v8bf& p2) __attribute__((always_inline)) {
      const char* vb = reinterpret_cast<const char*>(vt) + l16 * (2 * BN);
      auto load_op = [&](int i) __attribute__((always_inline)) -> v4i {
        if (i < 8) {
          const int k2 = i >> 2, c4 = i & 3;
          return *reinterpret_cast<const v4i*>(kt + (32 * s + 16 * k2 + rl) * D + koff[c4]);
        }
        const char* row = vb + (i - 8) * 16 * (2 * BN);
        const uint2 lo = *reinterpret_cast<const uint2*>(row + voff[s][0]);
        const uint2 hi = *reinterpret_cast<const uint2*>(row + voff[s][1]);
        return v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
      };
      constexpr int NOP = 24;
      constexpr int PD = SL8_Q16_PD;
      v4i opb[NOP];
#pragma unroll
      for (int i = 0; i < PD; ++i) opb[i] = load_op(i);
      __builtin_amdgcn_sched_barrier(0);
      const float tm0 = xmi * qsc;
      const bool ug = tm0 > m_run + a.w8_excess;
      const bool any_up = __any(ug);
      const float fr = ug ? __builtin_amdgcn_exp2f(m_run - tm0) : 1.f;
      if (ug) m_run = tm0;
      const bool any_key = tm0 != -INFINITY;
      const float sub = any_key ? tm0 - LOG2_127 : 0.f;
      const float fac = any_key ? __builtin_amdgcn_exp2f(tm0 - m_run) * (1.0f / 127.0f) : 0.f;
      float pe[8], py[8];
      float hs = 0.f, xm = -INFINITY;
      float4 kv[2];
      v4i sc[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
      // the P code of key e in two steps two MFMAs apart, so that the exp2
      // latency is covered: a: y = exp2(x q_scale - sub); b: the row sum,
      // rint and the scale
      auto pc_a = [&](int e) __attribute__((always_inline)) {
        py[e] = __builtin_amdgcn_exp2f(fmaf(xi[e], qsc, -sub));
        pin_vgpr(py[e]);
      };
      auto pc_b = [&](int e) __attribute__((always_inline)) {
        hs += py[e];
        pe[e] = rintf(py[e]) * fac;
        pin_vgpr(pe[e]);
        pin_vgpr(hs);
      };
      auto conv = [&](int e) __attribute__((always_inline)) {
        const float kk[4] = {kv[e >> 2].x, kv[e >> 2].y, kv[e >> 2].z, kv[e >> 2].w};
        xo[e] = (float)sc[e >> 2][e & 3] * kk[e & 3];
        pin_vgpr(xo[e]);
      };
      // slices: MFMA 0..7 (QK): P codes of keys 0..3 (a of key i / 2 after
      // MFMA i even, b after i + 1); MFMA 8 (PV 0): the k_scale reads;
      // MFMAs 9..16: the score of key i - 9 and the P codes of keys 4..7 the
      // same way; 17: pack P, l; 18: the scores' max in this lane; 19: across
      // the lane groups (xmo)
#pragma unroll
      for (int i = 0; i < NOP; ++i) {
        if (i + PD < NOP) opb[i + PD] = load_op(i + PD);
        __builtin_amdgcn_sched_barrier(0);
        if (i < 8) {
          sc[i >> 2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(opb[i], qop[i & 3], sc[i >> 2], 0, 0, 0);
          if (i & 1) pc_b(i >> 1);
          else pc_a(i >> 1);
        } else {
          const int tb = i - 8;
          oacc[tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, opb[i]), p2, oacc[tb], 0, 0, 0);
          if (i == 8) {
            kv[0] = *reinterpret_cast<const float4*>(st + 32 * s + kg);
            kv[1] = *reinterpret_cast<const float4*>(st + 32 * s + 16 + kg);
          } else if (i <= 16) {
            conv(i - 9);
            const int k = 4 + ((i - 9) >> 1);
            if ((i - 9) & 1) pc_b(k);
            else pc_a(k);
          } else if (i == 17) {
#pragma unroll
            for (int e = 0; e < 8; ++e) p1[e] = (__bf16)pe[e];
            pin_vgpr(__builtin_bit_cast(v4i, p1));
            l_lane = l_lane * fr + hs * fac;
          } else if (i == 18) {
#pragma unroll
            for (int e = 0; e < 8; ++e) xm = fmaxf(xm, xo[e]);
            pin_vgpr(xm);
          } else if (i == 19) {
            const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(xm), __float_as_uint(xm), false, false);
            xmo = max_xor32(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
            pin_vgpr(xmo);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (any_up) {
#pragma unroll
        for (int t = 0; t < 16; ++t) oacc[t] *= fr;
      }
    };
    // masked halves and halves that may fix a row's reference point
    auto half_fixup = [&](int t, int s, bool do_mask, bool dead, xblk16& xo, float& xmo)
        __attribute__((always_inline)) {
      if (do_mask) {
        const int nb = n_beg + t * BN + 32 * s;
        // key n is visible iff (n - lo) unsigned < (hi - lo)
        const int hi = dead ? nb : min(N, CAUSAL ? qpos + 1 : N);
        const int lo = (wl >= 0) ? qpos - wl + 1 : INT_MIN / 2;
        const int lo_c = max(lo, nb - 64);
        const uint32_t span = hi > lo_c ? (uint32_t)(hi - lo_c) : 0u;
        const uint32_t rel = (uint32_t)(nb + kg - lo_c);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          xo[e] = (rel + (uint32_t)(16 * (e >> 2) + (e & 3)) < span) ? xo[e] : -INFINITY;
      }
      xmo = row_max(xo);
      // the first visible half fixes the row's reference point
      if (m_run == -INFINITY && xmo != -INFINITY) m_run = xmo * qsc;
      all_set = !__any(m_run == -INFINITY);
    };
    auto body = [&](int j, const int8_t* kcur, int8_t* knext, uint16_t* vcopy, const uint16_t* vprev,
                    const float* scur, float* snext) __attribute__((always_inline)) {
      const int n0 = n_beg + j * BN;
      if (j + 1 < ntiles) {
        load_k(n0 + BN, knext);
        load_s(n0 + BN, snext);
      }
      const bool dead = !live(j);
      const bool mask = dead || masked(j);
      const bool skip = dead && !live(j - 1);  // nothing pending: P = 0, scores -inf
      if (!skip) {
        half_step_fast(0, kcur, scur, vprev, xB, xmB, pB, xA, xmA, pA);
        if (mask || !all_set) half_fixup(j, 0, mask, dead, xA, xmA);
      }
      if (j < ntiles) load_v(n0, vcopy);
      if (!skip) {
        half_step_fast(1, kcur, scur, vprev, xA, xmA, pA, xB, xmB, pB);
        if (mask || !all_set) half_fixup(j, 1, mask, dead, xB, xmB);
      }
      wait_dma();
      __syncthreads();
    };
    if (ntiles > 0) {
      load_k(n_beg, sk0);
      load_s(n_beg, ss0);
    }
    wait_dma();
    __syncthreads();
    int j = 0;
    for (; j + 1 <= ntiles; j += 2) {
      body(j, sk0, sk1, sv0, sv1, ss0, ss1);
      body(j + 1, sk1, sk0, sv1, sv0, ss1, ss0);
    }
    if (j <= ntiles) body(j, sk0, sk1, sv0, sv1, ss0, ss1);

    // l over the 4 lane groups of the query
    float l = l_lane;
    {
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(l), __float_as_uint(l), false, false);
      l = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
      l = __uint_as_float(r2[0]) + __uint_as_float(r2[1]);
    }
    if (m_ok) {
      const float inv = (l > 0.f) ? 1.f / l : 0.f;
      uint16_t* orow = reinterpret_cast<uint16_t*>(a.out) + ((int64_t)bh * M + mq) * a.dout;
#pragma unroll
      for (int tb = 0; tb < 16; ++tb) {
        const int d0 = 16 * tb + 4 * g;
        if (d0 >= a.dout) continue;  // zero-padded channels
        const float4 v4 = *reinterpret_cast<const float4*>(a.vs + bkv * D + d0);
        const float vsc[4] = {v4.x, v4.y, v4.z, v4.w};
        uint16_t hv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) hv[e] = f2h_bits(oacc[tb][e] * inv * vsc[e]);
        uint2 pk;
        pk.x = hv[0] | ((uint32_t)hv[1] << 16);
        pk.y = hv[2] | ((uint32_t)hv[3] << 16);
        *reinterpret_cast<uint2*>(orow + d0) = pk;
      }
    }
    __syncthreads();  // the next pass's first copies reuse the tiles
  }
}

}  // namespace

int w8a8_wide_launch(const int8_t* q, const float* q_scale, const int8_t* k, const float* k_scale,
                     const int8_t* v, const float* v_scale, void* out, int64_t B, int64_t Hq,
                     int64_t Hkv, int64_t M, int64_t N, int64_t D, int64_t dout, bool causal,
                     int64_t causal_diag, void* vt_ws, hipStream_t st) {
  uint16_t* vt = static_cast<uint16_t*>(vt_ws);
  if (N > 0) {
    const int np = (int)npad_of(N);
    const dim3 tg((unsigned)(np / 64), (unsigned)(B * Hkv));
    if (D == 64) v8_to_bf16_t_kernel<64><<<tg, 256, 0, st>>>(v, vt, (int)N, np);
    else if (D == 128) v8_to_bf16_t_kernel<128><<<tg, 256, 0, st>>>(v, vt, (int)N, np);
    else v8_to_bf16_t_kernel<256><<<tg, 256, 0, st>>>(v, vt, (int)N, np);
    SL8_CHECK_LAUNCH("attn_w8a8_fwd v to bf16 V^T");
  }
  int grid;
  FwdArgs a = make_args(B, Hq, Hkv, M, N, D, causal, grid);
  a.q = q; a.qs = q_scale; a.k = k; a.ks = k_scale;
  a.vt = vt; a.vs = v_scale; a.out = out; a.lse = nullptr;
  a.diag = (int)causal_diag;
  a.dout = (int)dout;
  a.w8_excess = w8_excess_for(N);
  constexpr int F = SL8_DTYPE_BF16;
  if (SL8_W8_Q16 && D == 256) {
    if (causal) attn_w8a8_q16_kernel<true><<<grid, 512, 0, st>>>(a);
    else attn_w8a8_q16_kernel<false><<<grid, 512, 0, st>>>(a);
  } else if (D == 64) {
    if (causal) launch_wide<64, true, F, false, true>(a, grid, st);
    else launch_wide<64, false, F, false, true>(a, grid, st);
  } else if (D == 128) {
    if (causal) launch_wide<128, true, F, false, true>(a, grid, st);
    else launch_wide<128, false, F, false, true>(a, grid, st);
  } else {
    if (causal) launch_wide<256, true, F, false, true>(a, grid, st);
    else launch_wide<256, false, F, false, true>(a, grid, st);
  }
  SL8_CHECK_LAUNCH("attn_w8a8_fwd");
  return SL8_OK;
}

}  // namespace sl8

using namespace sl8;

// The prefill reads V in place (natural layout): the workspace only holds the
// zero-padded operands of head dims 32, 72 and 80.
extern "C" size_t sl8_attn_int8_fwd_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t M,
                                              int64_t N, int64_t D) {
  return pad_workspace(B, Hq, Hkv, M, N, D, 2, false);
}

namespace {
int attn_int8_fwd_impl(const int8_t* q, const float* q_scale, const int8_t* k,
                       const float* k_scale, const void* v, int v_dtype, void* out, float* lse,
                       int64_t B, int64_t Hq, int64_t Hkv, int64_t M, int64_t N, int64_t D,
                       int causal, int64_t window_left, void* workspace, size_t workspace_bytes,
                       const int32_t* skip, void* stream) {
  int rc = check_fwd_shape(B, Hq, Hkv, M, N, D);
  if (rc) return rc;
  SL8_CHECK_ARG(v_dtype == SL8_DTYPE_F16 || v_dtype == SL8_DTYPE_BF16,
                "fni8: v must be float16 or bfloat16");
  SL8_CHECK_ARG(window_left >= -1 && window_left < (1LL << 30), "fni8: bad window_left");
  if (B == 0 || Hq == 0 || M == 0) return SL8_OK;
  SL8_CHECK_ARG(q && q_scale && out && (N == 0 || (k && k_scale && v)), "fni8: null pointer");
  SL8_CHECK_ARG(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(out, 16),
                "fni8: q/k/v/out must be 16-byte aligned");
  const size_t need = sl8_attn_int8_fwd_workspace(B, Hq, Hkv, M, N, D);
  SL8_CHECK_ARG(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 16)),
                "fni8: attn_int8_fwd workspace needs %zu bytes", need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t DP = padded_head_dim(D);
  if (DP != D) {
    Padded p;
    rc = pad_operands(q, k, v, nullptr, B, Hq, Hkv, M, N, D, 2, workspace, st, p);
    if (rc) return rc;
    q = p.q;
    k = p.k;
    v = p.v;
  }
  const bool c = causal != 0, want_lse = lse != nullptr;
  int grid;
  const int wv = wide_waves_for(DP, B, Hq, M, c);
  FwdArgs a = make_args(B, Hq, Hkv, M, N, DP, c, grid, wv);
  a.q = q; a.qs = q_scale; a.k = k; a.ks = k_scale;
  a.vt = static_cast<const uint16_t*>(v);  // V [B*Hkv][N][DP], read in place
  a.out = out; a.lse = lse; a.window_left = (int)window_left;
  a.dout = (int)D;
  a.skip = skip;
  const bool f16 = v_dtype == SL8_DTYPE_F16;
  if (DP == 64) {
    if (f16) dispatch_wide<64, SL8_DTYPE_F16>(a, grid, c, want_lse, wv, st);
    else dispatch_wide<64, SL8_DTYPE_BF16>(a, grid, c, want_lse, wv, st);
  } else if (DP == 128) {
    if (f16) dispatch_wide<128, SL8_DTYPE_F16>(a, grid, c, want_lse, wv, st);
    else dispatch_wide<128, SL8_DTYPE_BF16>(a, grid, c, want_lse, wv, st);
  } else {
    if (f16) dispatch_wide<256, SL8_DTYPE_F16>(a, grid, c, want_lse, wv, st);
    else dispatch_wide<256, SL8_DTYPE_BF16>(a, grid, c, want_lse, wv, st);
  }
  SL8_CHECK_LAUNCH("attn_int8_fwd");
  return SL8_OK;
}
}  // namespace

extern "C" int sl8_attn_int8_fwd(const int8_t* q, const float* q_scale, const int8_t* k,
                                 const float* k_scale, const void* v, int v_dtype, void* out,
                                 float* lse, int64_t B, int64_t Hq, int64_t Hkv, int64_t M,
                                 int64_t N, int64_t D, int causal, int64_t window_left,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return attn_int8_fwd_impl(q, q_scale, k, k_scale, v, v_dtype, out, lse, B, Hq, Hkv, M, N, D,
                            causal, window_left, workspace, workspace_bytes, nullptr, stream);
}

extern "C" int sl8_attn_int8_fwd_gated(const int8_t* q, const float* q_scale, const int8_t* k,
                                       const float* k_scale, const void* v, int v_dtype,
                                       void* out, float* lse, int64_t B, int64_t Hq, int64_t Hkv,
                                       int64_t M, int64_t N, int64_t D, int causal,
                                       int64_t window_left, void* workspace,
                                       size_t workspace_bytes, const int32_t* gate_flag,
                                       void* stream) {
  clear_error();
  SL8_CHECK_ARG(gate_flag != nullptr, "fni8: attn_int8_fwd_gated needs the gate flag");
  return attn_int8_fwd_impl(q, q_scale, k, k_scale, v, v_dtype, out, lse, B, Hq, Hkv, M, N, D,
                            causal, window_left, workspace, workspace_bytes, gate_flag, stream);
}

extern "C" int sl8_attn_int8_qk_scores(const int8_t* q, const int8_t* k, int32_t* scores,
                                       int64_t B, int64_t Hq, int64_t Hkv, int64_t M, int64_t N,
                                       int64_t D, int causal, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = check_fwd_shape(B, Hq, Hkv, M, N, D);
  if (rc) return rc;
  if (B == 0 || Hq == 0 || M == 0 || N == 0) return SL8_OK;
  SL8_CHECK_ARG(q && k && scores, "fni8: null pointer");
  SL8_CHECK_ARG(aligned(q, 16) && aligned(k, 16), "fni8: q/k must be 16-byte aligned");
  const size_t need = sl8_attn_int8_fwd_workspace(B, Hq, Hkv, M, N, D);
  SL8_CHECK_ARG(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 16)),
                "fni8: attn_int8_qk_scores workspace needs %zu bytes", need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t DP = padded_head_dim(D);
  if (DP != D) {  // zero channels add nothing to the int32 sums
    Padded p;
    rc = pad_operands(q, k, nullptr, nullptr, B, Hq, Hkv, M, N, D, 2, workspace, st, p);
    if (rc) return rc;
    q = p.q;
    k = p.k;
  }
  const bool c = causal != 0;
  int grid;
  FwdArgs a = make_args(B, Hq, Hkv, M, N, DP, c, grid);
  a.q = q; a.k = k; a.scores = scores;
  a.dout = (int)D;
  // V and the scales are never read by the dump instantiation
  constexpr int F = SL8_DTYPE_F16;
  if (DP == 64) {
    if (c) attn_fwd_wide_kernel<64, true, F, false, wide_ng(64), wide_waves(64), false, true>
        <<<grid, wide_waves(64) * 64, 0, st>>>(a);
    else attn_fwd_wide_kernel<64, false, F, false, wide_ng(64), wide_waves(64), false, true>
        <<<grid, wide_waves(64) * 64, 0, st>>>(a);
  } else if (DP == 128) {
    if (c) attn_fwd_wide_kernel<128, true, F, false, wide_ng(128), wide_waves(128), false, true>
        <<<grid, wide_waves(128) * 64, 0, st>>>(a);
    else attn_fwd_wide_kernel<128, false, F, false, wide_ng(128), wide_waves(128), false, true>
        <<<grid, wide_waves(128) * 64, 0, st>>>(a);
  } else {
    if (c) attn_fwd_wide_kernel<256, true, F, false, wide_ng(256), wide_waves(256), false, true>
        <<<grid, wide_waves(256) * 64, 0, st>>>(a);
    else attn_fwd_wide_kernel<256, false, F, false, wide_ng(256), wide_waves(256), false, true>
        <<<grid, wide_waves(256) * 64, 0, st>>>(a);
  }
  SL8_CHECK_LAUNCH("attn_int8_qk_scores");
  return SL8_OK;
}
