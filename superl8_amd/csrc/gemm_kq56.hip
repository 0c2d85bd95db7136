// GGUF Q5_K and Q6_K linear layers on native super-blocks, gfx950.
//
// Math (reference csrc/include/gemm_q4k_dp4a.cuh:200-489, the dp4a tile
// kernels, and csrc/include/gemm_decode_dp4a.cuh's decode variants):
//   Q5_K: y[m,n] = x_scale[m] * sum_j ( d*sc_j*<x_j, q_j> - dmin*m_j*sum(x_j) )
//         over 32-element sub-blocks j; q in [0,31] (4 bits in qs with
//         Q4_K's nibble interleave, the 5th bit in qh); sc_j, m_j 6-bit.
//   Q6_K: y[m,n] = x_scale[m] * sum_i d*sc_i*<x_i, q_i - 32>
//         over 16-element sub-blocks i; q in [0,63] (4 bits in ql, 2 in qh);
//         sc_i signed int8.
// x is the per-row int8 activation with its fp32 scale.
//
// Tile GEMM (M > 16; the decode GEMV below serves M <= 16): a 128 x 128 output
// tile per workgroup, the x tile and the 128 weight super-blocks copied
// global -> LDS one super-block ahead (double-buffered). Q5_K runs 8 waves,
// two per SIMD, each owning 32 output columns x 64 rows (each B operand built
// by the two waves of its columns); Q6_K, whose operand build costs the most,
// runs 4 waves, one per SIMD, each over 32 columns x all 128 rows (each B
// operand built once).
// The integer dot products stay exact:
//   Q5_K on v_mfma_i32_32x32x32_i8, one K = 32 step per sub-block: with
//     q = n + 16 b (n the low nibble, b the 5th bit), q * sc_j =
//     n (sc_j & 7) + 8 (n (sc_j >> 3) + 2 b sc_j), and each of the three B
//     operands n (sc & 7), n (sc >> 3), 2 b sc is at most 126, so it fits int8
//     (a 32-bit multiply scales 4 codes at once without carries). Three
//     MFMAs into T_lo, T_hi, T_hi; per super-block f += d * (T_lo + 8 T_hi).
//     The min term U = sum_j m_j * sum(x_j) on one fp16 MFMA per row block
//     and super-block (x half-sums x mins, exact), f -= dmin * U one
//     super-block later, as in the Q4_K tile kernel.
//   Q6_K on v_mfma_i32_32x32x32_i8 as well, one K = 32 step per pair of
//     16-element sub-blocks (each lane half holds one sub-block, so one scale
//     per lane): P = (q - 32) * sc in [-4096, 4064] is split exactly into two
//     int8 B operands, P = 256 B_hi + B_lo, two MFMAs into T_lo, T_hi, and
//     f += d * (T_lo + 256 T_hi) per super-block (details at the kernel).

#include "kquant.hpp"

namespace sl8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i_t __attribute__((ext_vector_type(16)));
typedef float v16f_t __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int Q5K_BYTES = 176;
constexpr int Q6K_BYTES = 210;
constexpr int KBM = 128, KBN = 128;                       // output tile
// full k-quant tiles on 8 waves (two per SIMD, RB = 2): config 4's shape at
// M = 512, same box, Q4_K 143 -> 123 us, Q5_K 174 -> 159 us; Q6_K, whose B
// operands cost the most VALU to build (each is then built by two waves),
// 186 -> 205 us, so it keeps 4 waves
#ifndef SL8_KQ_NW8
#define SL8_KQ_NW8 1
#endif
#ifndef SL8_Q6_NW8
#define SL8_Q6_NW8 0
#endif

// x tile copy by NT threads: 128 rows x 256 int8 of super-block sb; 16-byte
// chunk c of row r lands at r * 256 + 16 * (c ^ (r & 15)) (rows are one
// 256-byte bank line). QTR: rows 32 q .. 32 q + 31 only (a last-round
// quarter workgroup reads no other rows)
template <int NT, bool QTR>
__device__ __forceinline__ void copy_x_tile(const int8_t* x, int8_t* xd, int m0, int M, int K, int sb,
                                            int tid, int wave, int q = 0) {
  constexpr int XCH = QTR ? 512 : KBM * 16;
#pragma unroll
  for (int i = 0; i < XCH / NT; ++i) {
    const int P0 = (QTR ? q * 512 : 0) + i * NT;
    const int P = P0 + tid, row = P >> 4;
    const int c = (P & 15) ^ (row & 15);
    const int8_t* src = x + (int64_t)min(m0 + row, M - 1) * K + (int64_t)sb * 256 + 16 * c;
    __builtin_amdgcn_global_load_lds((kq_gptr_t)src, (kq_lptr_t)(xd + (P0 + wave * 64) * 16), 16, 0, 0);
  }
}

// ---------------------------------------------------------------------------
// Q5_K tile GEMM
// ---------------------------------------------------------------------------
// RB row blocks (32 rows) per wave, NW waves per workgroup, as the Q4_K tile
// kernel: full tiles RB = 2, NW = 8 (two waves per SIMD, each over 64 rows)
// or RB = 4, NW = 4; RB = 1, NW = 4 is a row quarter of a tile
template <int OUT_DT, int RB, int NW = 4>
__global__ void __launch_bounds__(64 * NW, 1)
gemm_q5k_tile_kernel(const int8_t* __restrict__ x, const float* __restrict__ x_scale,
                     const uint8_t* __restrict__ w, void* __restrict__ out, int M, int N, int K,
                     int nt_x, int xcd_m, int tile0) {
  constexpr bool QTR = RB * NW < 16;
  constexpr int NT = 64 * NW;
  constexpr int WCH = (KBN * 11 + NT - 1) / NT * NT;  // weight-tile 16-B chunks, whole copies
  __shared__ __attribute__((aligned(16))) int8_t xs0[KBM * 256];
  __shared__ __attribute__((aligned(16))) int8_t xs1[KBM * 256];
  __shared__ __attribute__((aligned(16))) uint8_t ws0[WCH * 16];
  __shared__ __attribute__((aligned(16))) uint8_t ws1[WCH * 16];
  // full tiles: the min-term MFMA's A operands (x half-sums) of one
  // super-block, [slot][row block][lane]; the scheme of the Q4_K tile kernel
  __shared__ __attribute__((aligned(16))) uint4 xh_l[QTR ? 1 : 2][QTR ? 1 : 4][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  // full tiles: one 128 x 128 tile per workgroup (tiles tile0, tile0 + 1, ...);
  // quarters: the quarter blockIdx.x & 3 (32 rows) of tile tile0 + blockIdx.x / 4,
  // so a short last round of tiles spreads over 4x the workgroups
  const int tile = tile0 + (QTR ? (int)(blockIdx.x >> 2) : (int)blockIdx.x);
  int ct, rt;
  kq_tile_coords(tile, nt_x, xcd_m, ct, rt);
  const int n0 = ct * KBN, m0 = rt * KBM;
  const int rb0 = QTR ? (int)(blockIdx.x & 3) : 0;
  const int cg = wave & 3;                                       // the wave's 32 output columns
  const int rbw = QTR ? rb0 : (NW == 8 ? (wave >> 2) * RB : 0);  // its first row block
  const int nsb = K >> 8;
  const int64_t row_bytes = (int64_t)nsb * Q5K_BYTES;

  auto load = [&](int sb, int8_t* xd, uint8_t* wd) __attribute__((always_inline)) {
    copy_x_tile<NT, QTR>(x, xd, m0, M, K, sb, tid, wave, rb0);
#pragma unroll
    for (int i = 0; i < WCH / NT; ++i) {
      const int P = min(i * NT + tid, KBN * 11 - 1), row = P / 11, c = P - 11 * row;
      const uint8_t* src = w + (int64_t)min(n0 + row, N - 1) * row_bytes + (int64_t)sb * Q5K_BYTES + 16 * c;
      __builtin_amdgcn_global_load_lds((kq_gptr_t)src, (kq_lptr_t)(wd + (i * NT + wave * 64) * 16), 16, 0, 0);
    }
  };

  // wave (cg, row group) owns weight rows 32 cg .. 32 cg + 31 (output
  // columns) for its RB row blocks; step j + 1's A reads and B operands are
  // formed while step j's MFMAs run (one scheduling region per step)
  float f[RB][16];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int e = 0; e < 16; ++e) f[rb][e] = 0.f;

  // min term U = sum_j m_j * xsum_j on one fp16 MFMA per row block and
  // super-block (exact: fp16 half-sums and mins, fp32 integer result); in a
  // full tile one super-block late through LDS, as in the Q4_K tile kernel
  float u_dmin = 0.f;
  v8h u_b = {}, u_a = {};  // its m_j operand and (quarters) its half-sum operand
  auto u_step = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const v8h a = QTR ? u_a : __builtin_bit_cast(v8h, xh_l[slot][rbw + rb][lane]);
      const v16f_t u = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, u_b, v16f_t{}, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 16; ++e) f[rb][e] -= u_dmin * u[e];
    }
  };

  // the half-sums this wave forms: row block urb, sub-blocks ju0 .. ju0 + JN - 1
  constexpr int JN = (NW == 8 && !QTR) ? 4 : 8;
  const int urb = QTR ? rb0 : (wave & 3);
  const int ju0 = (NW == 8 && !QTR) ? 4 * (wave >> 2) : 0;
  const int urow = 32 * urb + l32;

  auto compute = [&](const int8_t* xt, const uint8_t* wt, int slot) __attribute__((always_inline)) {
    const uint8_t* wr = wt + (32 * cg + l32) * Q5K_BYTES;
    const uint4 hd = *reinterpret_cast<const uint4*>(wr);
    const float d = h2f(hd.x & 0xFFFFu), dmin = h2f(hd.x >> 16);
    const ScMin sm = unpack_scmin(hd.y, hd.z, hd.w);
    const uint4 qhv = *reinterpret_cast<const uint4*>(wr + 16 + 16 * h);  // qh of l = 16h..16h+15
    const uint32_t qh[4] = {qhv.x, qhv.y, qhv.z, qhv.w};
    uint32_t qw[4][4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint4 qv = *reinterpret_cast<const uint4*>(wr + 48 + 32 * g + 16 * h);
      qw[g][0] = qv.x; qw[g][1] = qv.y; qw[g][2] = qv.z; qw[g][3] = qv.w;
    }
    float hsum[8];
    v4i A[2][RB], bl[2], bh[2], bb[2];
    auto read_a = [&](int j, int buf) __attribute__((always_inline)) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int row = 32 * (rbw + rb) + l32;
        A[buf][rb] = *reinterpret_cast<const v4i*>(xt + row * 256 + 16 * ((2 * j + h) ^ (row & 15)));
      }
    };
    // half-sum of sub-block ju0 + jj (jj < JN) of this lane's row urow, half h
    auto xsum_half = [&](int jj) __attribute__((always_inline)) {
      const int j = ju0 + jj;
      const v4i xv = QTR ? A[jj & 1][0]
                         : *reinterpret_cast<const v4i*>(xt + urow * 256 + 16 * ((2 * j + h) ^ (urow & 15)));
      int sacc = __builtin_amdgcn_sdot4(xv[0], 0x01010101, 0, false);
      sacc = __builtin_amdgcn_sdot4(xv[1], 0x01010101, sacc, false);
      sacc = __builtin_amdgcn_sdot4(xv[2], 0x01010101, sacc, false);
      sacc = __builtin_amdgcn_sdot4(xv[3], 0x01010101, sacc, false);
      hsum[jj] = (float)sacc;
    };
    auto build = [&](int j, int buf) __attribute__((always_inline)) {
      const uint32_t scw = j < 4 ? sm.sc_lo : sm.sc_hi;
      const uint32_t sc = (scw >> (8 * (j & 3))) & 0xFF;
      // q = n + 16 b (n the nibble, b the 5th bit): q * sc = n (sc & 7) +
      // 8 (n (sc >> 3) + 2 b sc); every B byte <= 126
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t nib = (qw[j >> 1][e] >> (4 * (j & 1))) & 0x0F0F0F0Fu;
        const uint32_t hb = (qh[e] >> j) & 0x01010101u;
        bl[buf][e] = (int)mul_bytes(nib, sc & 7);  // <= 15 * 7, 15 * 7 and 1 * 126 per byte
        bh[buf][e] = (int)mul_bytes(nib, sc >> 3);
        bb[buf][e] = (int)mul_bytes(hb, 2 * sc);
      }
    };
    v16i_t tl[RB], th[RB];
    read_a(0, 0);
    build(0, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = j & 1;
      __builtin_amdgcn_sched_barrier(0);
      if (j < 7) read_a(j + 1, c ^ 1);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        if (j == 0) {
          tl[rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[c][rb], bl[c], v16i_t{}, 0, 0, 0);
          th[rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[c][rb], bh[c], v16i_t{}, 0, 0, 0);
        } else {
          tl[rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[c][rb], bl[c], tl[rb], 0, 0, 0);
          th[rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[c][rb], bh[c], th[rb], 0, 0, 0);
        }
        th[rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[c][rb], bb[c], th[rb], 0, 0, 0);
      }
      if constexpr (JN == 8) xsum_half(j);
      else if (j & 1) xsum_half(j >> 1);
      if (j < 7) build(j + 1, c ^ 1);
      __builtin_amdgcn_sched_group_barrier(0x100, RB + (QTR ? 0 : 1), 0);  // the LDS reads first
#pragma unroll
      for (int k = 0; k < 3 * RB; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, RB == 4 ? 3 : 8, 0);  // VALU
      }
    }
    v8h ub;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      ub[jj] = (_Float16)(float)(((jj < 4 ? sm.mn_lo : sm.mn_hi) >> (8 * (jj & 3))) & 0xFF);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int e = 0; e < 16; ++e) f[rb][e] += d * (float)(tl[rb][e] + 8 * th[rb][e]);
    // the previous super-block's U (in a full tile its operands were published
    // before the barrier this compute follows), then this one's goes pending;
    // both launches apply the same operations in the same order
    if (slot >= 0) u_step(slot ^ 1);
    if constexpr (QTR) {
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) u_a[jj] = (_Float16)hsum[jj];
    } else if constexpr (JN == 8) {
      v8h ua;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) ua[jj] = (_Float16)hsum[jj];
      xh_l[slot & 1][urb][lane] = __builtin_bit_cast(uint4, ua);
    } else {
      typedef _Float16 v4h __attribute__((ext_vector_type(4)));
      v4h ua;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) ua[jj] = (_Float16)hsum[jj];
      reinterpret_cast<uint2*>(&xh_l[slot & 1][urb][lane])[ju0 >> 2] = __builtin_bit_cast(uint2, ua);
    }
    u_dmin = dmin;
    u_b = ub;
  };

  load(0, xs0, ws0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  int sb = 0;
  for (; sb + 1 < nsb; sb += 2) {
    load(sb + 1, xs1, ws1);
    compute(xs0, ws0, sb == 0 ? -2 : 0);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    if (sb + 2 < nsb) load(sb + 2, xs0, ws0);
    compute(xs1, ws1, 1);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
  }
  if (sb < nsb) {
    compute(xs0, ws0, sb == 0 ? -2 : 0);
    if constexpr (!QTR) __syncthreads();
  }
  u_step((nsb - 1) & 1);  // the last super-block's U

  const int n = n0 + 32 * cg + l32;
  // the row scales first, unconditionally (clamped rows): one wait, not one per element
  float xsv[RB][16];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      xsv[rb][e] = x_scale[min(m0 + 32 * (rbw + rb) + 8 * (e >> 2) + 4 * h + (e & 3), M - 1)];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + 32 * (rbw + rb) + 8 * (e >> 2) + 4 * h + (e & 3);
      if (m < M && n < N) st_out<OUT_DT>(out, (int64_t)m * N + n, f[rb][e] * xsv[rb][e]);
    }
}

// ---------------------------------------------------------------------------
// Q6_K tile GEMM
// ---------------------------------------------------------------------------
// Q6_K tile GEMM on v_mfma_i32_32x32x32_i8. Wave w owns the 32 weight rows
// 32 w .. 32 w + 31 (output columns) for all 128 activation rows, so each
// weight operand is built once per workgroup. One K = 32 step s of a
// super-block covers elements 32 s .. 32 s + 31 (ql half s / 4, quadrant
// s % 4); lane half h holds elements 32 s + 16 h .. +15 of its column, which
// are exactly sub-block i = 2 s + h, so one scale per lane and step. Per
// element P = (q - 32) * sc_i lies in [-4096, 4064]; P + 128 is formed in
// packed 16-bit lanes and split exactly as P = 256 B_hi + B_lo with
// B_hi = (P + 128) >> 8 in [-16, 16] (its high byte) and B_lo in [-128, 127]
// (its low byte minus 128), both int8 B operands: two MFMAs per step into
// T_lo, T_hi (|T| < 2^28 over a super-block), then
// f += d * (float)(T_lo + 256 T_hi) per super-block.
// Weight staging: row r's block of super-block sb is copied as the 14 aligned
// 16-byte pieces from its address rounded down to 16 (224 bytes cover the
// 210-byte block at any even misalignment) to LDS row r * 224; every piece
// starts before the block's last byte, so no read leaves the 16-byte granule
// of valid data.
typedef short v2s_t __attribute__((ext_vector_type(2)));
#ifndef SL8_Q6T_SCHED
#define SL8_Q6T_SCHED 1
#endif

// 16 bytes at byte offset b (even) of a dword array in LDS: aligned dword
// reads + v_alignbyte. The address is formed by indexing the array itself (no
// pointer-to-integer round trip), so the compiler keeps its provenance and
// does not wait for the other buffer's in-flight copies before the read.
__device__ __forceinline__ uint4 lds16_off(const uint32_t* w, int b) {
  const uint32_t* a = w + (b >> 2);
  const uint32_t sh = (uint32_t)(b & 3);
  const uint32_t d0 = a[0], d1 = a[1], d2 = a[2], d3 = a[3], d4 = a[4];
  return make_uint4(__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh),
                    __builtin_amdgcn_alignbyte(d3, d2, sh), __builtin_amdgcn_alignbyte(d4, d3, sh));
}

constexpr int Q6P16 = 224;                     // LDS pitch of a staged Q6_K block (14 pieces)
// weight-tile dwords: the KBN x 14 pieces rounded up to whole copies of NT
// threads (+ read slack)
template <int NT>
constexpr int t6w() { return (KBN * 14 + NT - 1) / NT * NT * 4 + 16; }

// 4 six-bit codes (bytes) -> the B_lo and B_hi bytes of (q - 32) * sc;
// off2 = 128 - 32 sc in both 16-bit lanes
__device__ __forceinline__ void q6_split4(uint32_t q, v2s_t sc2, v2s_t off2, uint32_t& lo, uint32_t& hi) {
  // bytes 0, 1 and 2, 3 of q into 16-bit lanes (selector byte 0x0C gives zero)
  const v2s_t e0 = __builtin_bit_cast(v2s_t, __builtin_amdgcn_perm(0u, q, 0x0C010C00u));
  const v2s_t e1 = __builtin_bit_cast(v2s_t, __builtin_amdgcn_perm(0u, q, 0x0C030C02u));
  const v2s_t p0 = e0 * sc2 + off2, p1 = e1 * sc2 + off2;  // P + 128, v_pk_mad_i16, exact
  const uint32_t u0 = __builtin_bit_cast(uint32_t, p0), u1 = __builtin_bit_cast(uint32_t, p1);
  lo = __builtin_amdgcn_perm(u1, u0, 0x06040200u) ^ 0x80808080u;  // low bytes - 128
  hi = __builtin_amdgcn_perm(u1, u0, 0x07050301u);                // high bytes
}

// RB row blocks per wave, NW waves per workgroup, as the Q4_K tile kernel
template <int OUT_DT, int RB, int NW = 4>
__global__ void __launch_bounds__(64 * NW, 1)
gemm_q6k_tile_kernel(const int8_t* __restrict__ x, const float* __restrict__ x_scale,
                     const uint8_t* __restrict__ w, void* __restrict__ out, int M, int N, int K,
                     int nt_x, int xcd_m, int tile0) {
  constexpr bool QTR = RB * NW < 16;
  constexpr int NT = 64 * NW;
  __shared__ __attribute__((aligned(16))) int8_t xs0[KBM * 256];
  __shared__ __attribute__((aligned(16))) int8_t xs1[KBM * 256];
  __shared__ __attribute__((aligned(16))) uint32_t ws0[t6w<NT>()];
  __shared__ __attribute__((aligned(16))) uint32_t ws1[t6w<NT>()];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  // full tiles: one 128 x 128 tile per workgroup (tiles tile0, tile0 + 1, ...);
  // quarters: the quarter blockIdx.x & 3 (32 rows) of tile tile0 + blockIdx.x / 4,
  // so a short last round of tiles spreads over 4x the workgroups
  const int tile = tile0 + (QTR ? (int)(blockIdx.x >> 2) : (int)blockIdx.x);
  int ct, rt;
  kq_tile_coords(tile, nt_x, xcd_m, ct, rt);
  const int n0 = ct * KBN, m0 = rt * KBM;
  const int rb0 = QTR ? (int)(blockIdx.x & 3) : 0;
  const int cg = wave & 3;                                       // the wave's 32 output columns
  const int rbw = QTR ? rb0 : (NW == 8 ? (wave >> 2) * RB : 0);  // its first row block
  const int nsb = K >> 8;
  const int64_t row_bytes = (int64_t)nsb * Q6K_BYTES;
  const int rmax = min(KBN, N - n0) - 1;

  // piece P = NT i + tid of the weight tile: row P / 14, piece P % 14 (fixed
  // per thread; pieces past the tile, from rounding up to whole copies,
  // re-read the last row into the padding); offsets are 32-bit from the
  // workgroup's row-n0 base, which is 256-byte aligned (n0 of 128, row_bytes
  // even): 128 rows of < 2^24 bytes
  const uint8_t* wbase = w + (int64_t)n0 * row_bytes;
  auto load = [&](int sb, int8_t* xd, uint32_t* wd) __attribute__((always_inline)) {
    copy_x_tile<NT, QTR>(x, xd, m0, M, K, sb, tid, wave, rb0);
    const uint32_t sboff = (uint32_t)sb * Q6K_BYTES;
#pragma unroll
    for (int i = 0; i < (KBN * 14 + NT - 1) / NT; ++i) {
      const int P = i * NT + tid, Pc = min(P, KBN * 14 - 1), row = Pc / 14, c = Pc - 14 * (Pc / 14);
      const uint32_t off = (((uint32_t)min(row, rmax) * (uint32_t)row_bytes + sboff) & ~15u) + 16u * (uint32_t)c;
      __builtin_amdgcn_global_load_lds((kq_gptr_t)(wbase + off), (kq_lptr_t)(wd + (i * NT + wave * 64) * 4), 16, 0, 0);
    }
  };

  float f[RB][16];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int e = 0; e < 16; ++e) f[rb][e] = 0.f;

  const int r = 32 * cg + l32;  // this lane's weight row in the tile
  auto compute = [&](int sb, const int8_t* xt, const uint32_t* wt) __attribute__((always_inline)) {
    // the block's misalignment is that of its offset from the row-n0 base
    const uint32_t base = (uint32_t)min(r, rmax) * (uint32_t)row_bytes + (uint32_t)sb * Q6K_BYTES;
    const int blk = r * Q6P16 + (int)(base & 15u);  // byte offset of the block in the tile
    const uint4 scv = lds16_off(wt, blk + 192);
    const float d = h2f((uint16_t)(__builtin_amdgcn_alignbyte(wt[((blk + 208) >> 2) + 1], wt[(blk + 208) >> 2],
                                                             (uint32_t)((blk + 208) & 3)) & 0xFFFFu));
    v16i_t tl[RB], th[RB];
    // software pipeline over the 8 K steps: step s + 1's A reads and B
    // operands are formed while step s's 8 MFMAs run (double-buffered
    // registers; one scheduling region per step, MFMAs interleaved with VALU)
    uint32_t qv[2][12];  // ql quadrants 0/2, 1/3 and qh of each ql half
    auto load_q = [&](int hf) __attribute__((always_inline)) {
      const uint4 qa = lds16_off(wt, blk + 64 * hf + 16 * h);       // quadrants 0, 2
      const uint4 qb = lds16_off(wt, blk + 64 * hf + 32 + 16 * h);  // quadrants 1, 3
      const uint4 qc = lds16_off(wt, blk + 128 + 32 * hf + 16 * h);
      qv[hf][0] = qa.x; qv[hf][1] = qa.y; qv[hf][2] = qa.z; qv[hf][3] = qa.w;
      qv[hf][4] = qb.x; qv[hf][5] = qb.y; qv[hf][6] = qb.z; qv[hf][7] = qb.w;
      qv[hf][8] = qc.x; qv[hf][9] = qc.y; qv[hf][10] = qc.z; qv[hf][11] = qc.w;
    };
    v4i bl[2], bh[2], A[2][RB];
    auto build = [&](int s, int buf) __attribute__((always_inline)) {
      const int hf = s >> 2, qd = s & 3, i = 2 * s + h;  // ql half, quadrant, sub-block (scale index)
      const uint32_t sw = (s >> 1) == 0 ? scv.x : (s >> 1) == 1 ? scv.y : (s >> 1) == 2 ? scv.z : scv.w;
      const int sc = (int)(int8_t)(sw >> (8 * (i & 3)));
      const v2s_t sc2 = {(short)sc, (short)sc}, off2 = {(short)(128 - 32 * sc), (short)(128 - 32 * sc)};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t ql = qv[hf][4 * (qd & 1) + e];
        const uint32_t q = ((ql >> (4 * (qd >> 1))) & 0x0F0F0F0Fu) | (((qv[hf][8 + e] >> (2 * qd)) & 0x03030303u) << 4);
        uint32_t lo, hi;
        q6_split4(q, sc2, off2, lo, hi);
        bl[buf][e] = (int)lo;
        bh[buf][e] = (int)hi;
      }
    };
    auto read_a = [&](int s, int buf) __attribute__((always_inline)) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int row = 32 * (rbw + rb) + l32;
        A[buf][rb] = *reinterpret_cast<const v4i*>(xt + row * 256 + 16 * ((2 * s + h) ^ (row & 15)));
      }
    };
    load_q(0);
    read_a(0, 0);
    build(0, 0);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int c = s & 1;
#if SL8_Q6T_SCHED
      __builtin_amdgcn_sched_barrier(0);
#endif
      if (s == 1) load_q(1);
      if (s < 7) read_a(s + 1, c ^ 1);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        if (s == 0) {
          tl[rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[c][rb], bl[c], v16i_t{}, 0, 0, 0);
          th[rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[c][rb], bh[c], v16i_t{}, 0, 0, 0);
        } else {
          tl[rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[c][rb], bl[c], tl[rb], 0, 0, 0);
          th[rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[c][rb], bh[c], th[rb], 0, 0, 0);
        }
      }
      if (s < 7) build(s + 1, c ^ 1);
#if SL8_Q6T_SCHED
      __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // the LDS reads first
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // 6 VALU
      }
#endif
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int e = 0; e < 16; ++e) f[rb][e] += d * (float)(tl[rb][e] + 256 * th[rb][e]);
  };

  load(0, xs0, ws0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  int sb = 0;
  for (; sb + 1 < nsb; sb += 2) {
    load(sb + 1, xs1, ws1);
    compute(sb, xs0, ws0);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    if (sb + 2 < nsb) load(sb + 2, xs0, ws0);
    compute(sb + 1, xs1, ws1);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
  }
  if (sb < nsb) compute(sb, xs0, ws0);

  const int n = n0 + r;
  // the row scales first, unconditionally (clamped rows): one wait, not one per element
  float xsv[RB][16];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      xsv[rb][e] = x_scale[min(m0 + 32 * (rbw + rb) + 8 * (e >> 2) + 4 * h + (e & 3), M - 1)];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + 32 * (rbw + rb) + 8 * (e >> 2) + 4 * h + (e & 3);
      if (m < M && n < N) st_out<OUT_DT>(out, (int64_t)m * N + n, f[rb][e] * xsv[rb][e]);
    }
}

// ---------------------------------------------------------------------------
// Dequantisation to fp32 (checking and conversion helper)
// ---------------------------------------------------------------------------
__global__ void dequant_q5k_kernel(const uint8_t* __restrict__ w, float* __restrict__ out,
                                   int64_t N, int K) {
  const int nsub = K >> 5, nsb = K >> 8;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N * nsub) return;
  const int64_t n = t / nsub;
  const int js = (int)(t % nsub), sb = js >> 3, j = js & 7;
  const uint8_t* b = w + (n * nsb + sb) * Q5K_BYTES;
  const uint32_t* hd = reinterpret_cast<const uint32_t*>(b);
  const float d = h2f(hd[0] & 0xFFFFu), dmin = h2f(hd[0] >> 16);
  const ScMin sm = unpack_scmin(hd[1], hd[2], hd[3]);
  const uint32_t sc = byte_of(j < 4 ? sm.sc_lo : sm.sc_hi, j & 3);
  const uint32_t mn = byte_of(j < 4 ? sm.mn_lo : sm.mn_hi, j & 3);
  const float dsc = d * (float)sc, dm = dmin * (float)mn;
  float* o = out + n * K + (int64_t)js * 32;
  for (int l = 0; l < 32; ++l) {
    const int q = ((b[48 + 32 * (j >> 1) + l] >> (4 * (j & 1))) & 15) | (((b[16 + l] >> j) & 1) << 4);
    o[l] = __fsub_rn(__fmul_rn(dsc, (float)q), dm);  // two roundings, as the reference decoder
  }
}

__global__ void dequant_q6k_kernel(const uint8_t* __restrict__ w, float* __restrict__ out,
                                   int64_t N, int K) {
  const int nsub = K >> 4, nsb = K >> 8;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N * nsub) return;
  const int64_t n = t / nsub;
  const int is = (int)(t % nsub), sb = is >> 4, i = is & 15;
  const uint8_t* b = w + (n * nsb + sb) * Q6K_BYTES;
  const float d = h2f((uint16_t)(b[208] | (b[209] << 8)));
  const float rs = d * (float)(int8_t)b[192 + i];
  const int g = i >> 3, qd = (i & 7) >> 1, l0 = 16 * (i & 1);
  float* o = out + n * K + (int64_t)is * 16;
  for (int l = l0; l < l0 + 16; ++l) {
    const int qlb = b[64 * g + 32 * (qd & 1) + l];
    const int q = ((qlb >> (4 * (qd >> 1))) & 15) | (((b[128 + 32 * g + l] >> (2 * qd)) & 3) << 4);
    o[l - l0] = __fmul_rn(rs, (float)(q - 32));
  }
}

// ---------------------------------------------------------------------------
// Decode GEMV (M <= 16): one wave per weight row (two rows from M = 4 on,
// sharing every activation load), the lanes over units of 64 weights (4 per
// super-block: Q5_K sub-block pair g, Q6_K half g >> 1 x ql column g & 1),
// the dot products on VALU v_dot4 in registers; a fixed-order wave reduction
// keeps the output deterministic. Q6_K fields start on 2-byte
// boundaries: they are read as dword-aligned loads and v_alignbyte.
// ---------------------------------------------------------------------------
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));

// 8 dwords starting at a 2-byte aligned global address (9 aligned dwords + v_alignbyte)
__device__ __forceinline__ void load8_a2(const uint8_t* p, uint32_t (&o)[8]) {
  const uintptr_t ad = reinterpret_cast<uintptr_t>(p);
  const uint32_t* a = reinterpret_cast<const uint32_t*>(p - (ad & 3));  // keeps the global address space
  const uint32_t sh = (uint32_t)(ad & 3);
  const u32x4a d0 = *reinterpret_cast<const u32x4a*>(a);
  const u32x4a d1 = *reinterpret_cast<const u32x4a*>(a + 4);
  const uint32_t d8 = a[8];
  const uint32_t d[9] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w, d8};
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = __builtin_amdgcn_alignbyte(d[e + 1], d[e], sh);
}

// The 64 weights of one unit, unpacked (codes as int8 lanes of dwords) with
// their scales.
template <int FMT> struct UnitCodes;
template <> struct UnitCodes<5> {
  uint32_t c[2][8];       // sub-blocks 2g, 2g + 1: codes 0..31
  int sc[2], mn[2];
  float d, dmin;
};
template <> struct UnitCodes<6> {
  uint32_t c[2][8];       // quadrants p, p + 2: q - 32 as int8
  int sc[2][2];           // [quadrant][16-element half]
  float d;
};

__device__ __forceinline__ void unit_codes(const uint8_t* blk, int g, UnitCodes<5>& u) {
  // sub-blocks j0 = 2g (low nibbles) and j1 = 2g + 1 (high nibbles)
  const uint4 hd = *reinterpret_cast<const uint4*>(blk);
  const uint4 qh0 = *reinterpret_cast<const uint4*>(blk + 16);
  const uint4 qh1 = *reinterpret_cast<const uint4*>(blk + 32);
  const uint4 qs0 = *reinterpret_cast<const uint4*>(blk + 48 + 32 * g);
  const uint4 qs1 = *reinterpret_cast<const uint4*>(blk + 64 + 32 * g);
  u.d = h2f(hd.x & 0xFFFFu);
  u.dmin = h2f(hd.x >> 16);
  const ScMin sm = unpack_scmin(hd.y, hd.z, hd.w);
  const int j0 = 2 * g, j1 = j0 + 1;
  const uint32_t scw = g < 2 ? sm.sc_lo : sm.sc_hi, mnw = g < 2 ? sm.mn_lo : sm.mn_hi;
  u.sc[0] = byte_of(scw, j0 & 3);
  u.sc[1] = byte_of(scw, j1 & 3);
  u.mn[0] = byte_of(mnw, j0 & 3);
  u.mn[1] = byte_of(mnw, j1 & 3);
  const uint32_t qs[8] = {qs0.x, qs0.y, qs0.z, qs0.w, qs1.x, qs1.y, qs1.z, qs1.w};
  const uint32_t qh[8] = {qh0.x, qh0.y, qh0.z, qh0.w, qh1.x, qh1.y, qh1.z, qh1.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    u.c[0][e] = (qs[e] & 0x0F0F0F0Fu) | (((qh[e] >> j0) & 0x01010101u) << 4);
    u.c[1][e] = ((qs[e] >> 4) & 0x0F0F0F0Fu) | (((qh[e] >> j1) & 0x01010101u) << 4);
  }
}

__device__ __forceinline__ void unit_codes(const uint8_t* blk, int g, UnitCodes<6>& u) {
  // half hf = g >> 1, ql column p = g & 1: quadrants qd = p (low nibbles)
  // and p + 2 (high nibbles), l = 0..31 each
  const int hf = g >> 1, p = g & 1;
  uint32_t ql[8], qh[8];
  load8_a2(blk + 64 * hf + 32 * p, ql);
  load8_a2(blk + 128 + 32 * hf, qh);
  const uintptr_t sa = reinterpret_cast<uintptr_t>(blk + 192 + 8 * hf);
  const uint32_t* sp = reinterpret_cast<const uint32_t*>(blk + 192 + 8 * hf - (sa & 3));
  const uint32_t ssh = (uint32_t)(sa & 3);
  const uint32_t s0w = __builtin_amdgcn_alignbyte(sp[1], sp[0], ssh);  // scales 8hf + 0..3
  // (sp[2] only when the scales are misaligned: for an aligned block it lies
  // past the block's end)
  const uint32_t s1w = __builtin_amdgcn_alignbyte(sp[ssh ? 2 : 1], sp[1], ssh);  // scales 8hf + 4..7
  u.d = h2f(*reinterpret_cast<const uint16_t*>(blk + 208));
  u.sc[0][0] = (int)(int8_t)byte_of(s0w, 2 * p);
  u.sc[0][1] = (int)(int8_t)byte_of(s0w, 2 * p + 1);
  u.sc[1][0] = (int)(int8_t)byte_of(s1w, 2 * p);
  u.sc[1][1] = (int)(int8_t)byte_of(s1w, 2 * p + 1);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int qd = p + 2 * k;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t q = ((ql[e] >> (4 * k)) & 0x0F0F0F0Fu) | (((qh[e] >> (2 * qd)) & 0x03030303u) << 4);
      const uint32_t t = q ^ 0x20202020u;                // 6-bit two's complement of q - 32
      u.c[k][e] = t | ((t & 0x20202020u) * 6u);          // sign-extended to 8 bits
    }
  }
}

// The unit's 64 activations of one row: Q5_K elements 64g..64g+63 of the
// super-block; Q6_K quadrants p and p + 2 of half g >> 1 (32 each).
template <int FMT>
__device__ __forceinline__ void unit_x(const int8_t* xsb, int g, uint32_t (&v)[2][8]) {
  const int8_t* a = FMT == 5 ? xsb + 64 * g : xsb + 128 * (g >> 1) + 32 * (g & 1);
  const int8_t* b = FMT == 5 ? a + 32 : a + 64;
  const uint4 a0 = reinterpret_cast<const uint4*>(a)[0], a1 = reinterpret_cast<const uint4*>(a)[1];
  const uint4 b0 = reinterpret_cast<const uint4*>(b)[0], b1 = reinterpret_cast<const uint4*>(b)[1];
  v[0][0] = a0.x; v[0][1] = a0.y; v[0][2] = a0.z; v[0][3] = a0.w;
  v[0][4] = a1.x; v[0][5] = a1.y; v[0][6] = a1.z; v[0][7] = a1.w;
  v[1][0] = b0.x; v[1][1] = b0.y; v[1][2] = b0.z; v[1][3] = b0.w;
  v[1][4] = b1.x; v[1][5] = b1.y; v[1][6] = b1.z; v[1][7] = b1.w;
}

// sums of the unit's two 32-activation sub-blocks (the Q5_K min term)
__device__ __forceinline__ void unit_xsum(const uint32_t (&x)[2][8], int (&xs)[2]) {
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    xs[k] = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) xs[k] = __builtin_amdgcn_sdot4((int)x[k][e], 0x01010101, xs[k], false);
  }
}

__device__ __forceinline__ float unit_dot(const UnitCodes<5>& u, const uint32_t (&x)[2][8],
                                          const int (&xs)[2]) {
  int s[2] = {0, 0};
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) s[k] = __builtin_amdgcn_sdot4((int)x[k][e], (int)u.c[k][e], s[k], false);
  return u.d * (float)(u.sc[0] * s[0] + u.sc[1] * s[1]) - u.dmin * (float)(u.mn[0] * xs[0] + u.mn[1] * xs[1]);
}

__device__ __forceinline__ float unit_dot(const UnitCodes<5>& u, const uint32_t (&x)[2][8]) {
  int xs[2];
  unit_xsum(x, xs);
  return unit_dot(u, x, xs);
}

__device__ __forceinline__ float unit_dot(const UnitCodes<6>& u, const uint32_t (&x)[2][8]) {
  int T = 0;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s0 = __builtin_amdgcn_sdot4((int)x[k][e], (int)u.c[k][e], s0, false);
      s1 = __builtin_amdgcn_sdot4((int)x[k][4 + e], (int)u.c[k][4 + e], s1, false);
    }
    T += u.sc[k][0] * s0 + u.sc[k][1] * s1;
  }
  return u.d * (float)T;
}

// M = 2 (M = 1 runs gemv_kq_flat_kernel, M >= 3 the MFMA kernels): one wave
// per weight row (R rows per wave share every activation load), lanes over
// the row's units.
template <int FMT, int OUT_DT, int MR, int R>
__global__ void __launch_bounds__(256)
gemv_kq_kernel(const int8_t* __restrict__ x, const float* __restrict__ x_scale,
               const uint8_t* __restrict__ w, void* __restrict__ out, int M, int N, int K) {
  constexpr int BS = FMT == 5 ? Q5K_BYTES : Q6K_BYTES;
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  if (n0 >= N) return;  // wave-uniform
  const int nsb = K >> 8, nu = 4 * nsb;
  const int64_t row_bytes = (int64_t)nsb * BS;
  float f[R][MR];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) f[r][m] = 0.f;

  for (int u = lane; u < nu; u += 64) {
    const int sb = u >> 2, g = u & 3;
    UnitCodes<FMT> cd[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (n0 + r < N) unit_codes(w + (int64_t)(n0 + r) * row_bytes + (int64_t)sb * BS, g, cd[r]);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m < M) {
        uint32_t xv[2][8];
        unit_x<FMT>(x + (int64_t)m * K + (int64_t)sb * 256, g, xv);
        if constexpr (FMT == 5) {
          int xs[2];  // shared by the R weight rows
          unit_xsum(xv, xs);
#pragma unroll
          for (int r = 0; r < R; ++r)
            if (n0 + r < N) f[r][m] += unit_dot(cd[r], xv, xs);
        } else {
#pragma unroll
          for (int r = 0; r < R; ++r)
            if (n0 + r < N) f[r][m] += unit_dot(cd[r], xv);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) f[r][m] += __shfl_xor(f[r][m], o, 64);
    }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < M && n0 + r < N) st_out<OUT_DT>(out, (int64_t)m * N + n0 + r, f[r][m] * x_scale[m]);
  }
}

// M = 1: RF weight rows per wave with their units laid end to end over the
// lanes (K = 5120: 4 rows x 80 units = 5 full passes of 64 lanes, where one row
// per wave leaves 48 of 64 lanes idle in its second pass).
template <int FMT, int OUT_DT, int RF>
__global__ void __launch_bounds__(256)
gemv_kq_flat_kernel(const int8_t* __restrict__ x, const float* __restrict__ x_scale,
                    const uint8_t* __restrict__ w, void* __restrict__ out, int N, int K) {
  constexpr int BS = FMT == 5 ? Q5K_BYTES : Q6K_BYTES;
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RF;
  if (n0 >= N) return;  // wave-uniform
  const int nsb = K >> 8, nu = 4 * nsb;
  const int nr = min(RF, N - n0);
  const int64_t row_bytes = (int64_t)nsb * BS;
  float f[RF];
#pragma unroll
  for (int r = 0; r < RF; ++r) f[r] = 0.f;
  for (int v = lane; v < nr * nu; v += 64) {
    const int r = v / nu, u = v - r * nu;
    const int sb = u >> 2, g = u & 3;
    UnitCodes<FMT> cd;
    unit_codes(w + (int64_t)(n0 + r) * row_bytes + (int64_t)sb * BS, g, cd);
    uint32_t xv[2][8];
    unit_x<FMT>(x + (int64_t)sb * 256, g, xv);
    const float val = unit_dot(cd, xv);
#pragma unroll
    for (int rr = 0; rr < RF; ++rr) f[rr] += (rr == r) ? val : 0.f;
  }
#pragma unroll
  for (int r = 0; r < RF; ++r) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) f[r] += __shfl_xor(f[r], o, 64);
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < RF; ++r)
      if (r < nr) st_out<OUT_DT>(out, (int64_t)(n0 + r), f[r] * x_scale[0]);
  }
}

template <int FMT, int MR>
void launch_gemv_kq_m(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                      int M, int N, int K, hipStream_t st) {
  if (MR == 1) {
    constexpr int RF = FMT == 5 ? 4 : 2;  // measured at K = 5120: Q6_K's larger unit state favours 2
    const dim3 g1((unsigned)((N + 4 * RF - 1) / (4 * RF)));
    switch (odt) {
      case SL8_DTYPE_F16: gemv_kq_flat_kernel<FMT, SL8_DTYPE_F16, RF><<<g1, 256, 0, st>>>(x, xs, w, out, N, K); break;
      case SL8_DTYPE_BF16: gemv_kq_flat_kernel<FMT, SL8_DTYPE_BF16, RF><<<g1, 256, 0, st>>>(x, xs, w, out, N, K); break;
      default: gemv_kq_flat_kernel<FMT, SL8_DTYPE_F32, RF><<<g1, 256, 0, st>>>(x, xs, w, out, N, K); break;
    }
    return;
  }
  constexpr int R = 1;
  const dim3 grid((unsigned)((N + 4 * R - 1) / (4 * R)));
  switch (odt) {
    case SL8_DTYPE_F16: gemv_kq_kernel<FMT, SL8_DTYPE_F16, MR, R><<<grid, 256, 0, st>>>(x, xs, w, out, M, N, K); break;
    case SL8_DTYPE_BF16: gemv_kq_kernel<FMT, SL8_DTYPE_BF16, MR, R><<<grid, 256, 0, st>>>(x, xs, w, out, M, N, K); break;
    default: gemv_kq_kernel<FMT, SL8_DTYPE_F32, MR, R><<<grid, 256, 0, st>>>(x, xs, w, out, M, N, K); break;
  }
}

// ---------------------------------------------------------------------------
// Q6_K decode GEMV for 3 <= M <= 16 on the int8 MFMA (v_mfma_i32_16x16x64_i8).
// For ql half hf and nibble nb, the 16 k-slots of lane group h of one MFMA
// are exactly one 16-element sub-block: elements 128 hf + 64 nb + 16 h + 0..15
// (quadrant (h >> 1) + 2 nb, half-quadrant h & 1), with scale index
// 8 hf + 4 nb + h. A-operand row i = 4 g + mm carries activation row mm (of
// a block of 4) on the k-slots of group g only (zeros elsewhere), so the C
// rows 4 g .. 4 g + 3 a lane holds are the sub-block sums of its own group
// g = lane / 16 for 4 activation rows. B = q - 32 (6-bit codes, exact in
// int8). 16 weight rows per workgroup, the K range split over Q6W waves of
// up to Q6CH super-blocks; a lane 4 r + c loads 16-byte piece c of each
// 64-byte part (ql halves, qh) of weight row r. Q6_K blocks are 210 bytes,
// so odd super-blocks start 2 bytes off a dword: pieces are read as 5
// aligned dwords and v_alignbyte.
// ---------------------------------------------------------------------------
#ifndef SL8_Q6W  // measured at config 4's shape, M = 8: 8 x 3 27.6 us, 10 x 2 33.9, 5 x 4 34.3, 6 x 4 34.2
#define SL8_Q6W 8
#define SL8_Q6CH 3
#endif
constexpr int Q6W = SL8_Q6W, Q6CH = SL8_Q6CH;
constexpr int Q6XP = Q6CH * 256;  // LDS bytes per activation row and wave

__device__ __forceinline__ uint32_t q6_pull(uint32_t v, int src_lane) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src_lane << 2, (int)v);
}
// 16 bytes at a 2-byte aligned address (shift 0 or 2 from its aligned dword)
__device__ __forceinline__ uint4 load16_a2(const uint8_t* p, uint32_t sh) {
  const uint32_t* a = reinterpret_cast<const uint32_t*>(reinterpret_cast<uintptr_t>(p) & ~(uintptr_t)3);
  const u32x4a d = *reinterpret_cast<const u32x4a*>(a);
  const uint32_t e = a[4];
  return make_uint4(__builtin_amdgcn_alignbyte(d.y, d.x, sh), __builtin_amdgcn_alignbyte(d.z, d.y, sh),
                    __builtin_amdgcn_alignbyte(d.w, d.z, sh), __builtin_amdgcn_alignbyte(e, d.w, sh));
}

template <int OUT_DT, int MB>  // MB blocks of 4 activation rows
__global__ void __launch_bounds__(64 * Q6W)
gemv_q6k_mfma_kernel(const int8_t* __restrict__ x, const float* __restrict__ x_scale,
                     const uint8_t* __restrict__ w, void* __restrict__ out, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(16))) int8_t xq6[];  // per wave: M rows + a zero row
  __shared__ float red6[Q6W - 1][MB][16][4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nsb = K >> 8;
  const int lj = lane & 15, h = lane >> 4;   // operand column / k-group (= C-row group)
  const int lr = lane >> 2, lc = lane & 3;   // load role: weight row, 16-byte piece
  const int n0 = blockIdx.x * 16;
  const int64_t row_bytes = (int64_t)nsb * Q6K_BYTES;
  const uint8_t* wrow = w + (int64_t)min(n0 + lr, N - 1) * row_bytes;
  const int gA = lj >> 2, mA = lj & 3;       // A row lj = 4 gA + mA
  const int xarea = (M * Q6XP + 1023) & ~1023;
  int8_t* xw = xq6 + (int64_t)wave * (xarea + Q6XP);
  int8_t* xz = xw + xarea;                   // zero row
  for (int i = lane; i < Q6XP / 16; i += 64) reinterpret_cast<uint4*>(xz)[i] = make_uint4(0, 0, 0, 0);
  const int8_t* xrow[MB];
#pragma unroll
  for (int t = 0; t < MB; ++t) xrow[t] = (gA == h && 4 * t + mA < M) ? xw + (4 * t + mA) * Q6XP : xz;

  float f[MB][4];
#pragma unroll
  for (int t = 0; t < MB; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) f[t][r] = 0.f;

  auto chunk = [&](const int c0, const int cnt) {
    uint4 qlp[Q6CH][2], qhp[Q6CH];
    uint32_t scw[Q6CH], dw[Q6CH];
#pragma unroll
    for (int i = 0; i < Q6CH; ++i) {
      const int sb = min(c0 + i, nsb - 1);
      const uint8_t* blk = wrow + (int64_t)sb * Q6K_BYTES;
      const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3);
      qlp[i][0] = load16_a2(blk + 16 * lc, sh);
      qlp[i][1] = load16_a2(blk + 64 + 16 * lc, sh);
      qhp[i] = load16_a2(blk + 128 + 16 * lc, sh);
      const uint32_t* sp = reinterpret_cast<const uint32_t*>(reinterpret_cast<uintptr_t>(blk + 192 + 4 * lc) & ~(uintptr_t)3);
      // sp[1] only when misaligned (aligned: it lies past the block for lc = 3);
      // d by a 16-bit load (2-byte aligned), never past the block
      scw[i] = __builtin_amdgcn_alignbyte(sp[sh ? 1 : 0], sp[0], sh);  // scales 4 lc .. 4 lc + 3
      dw[i] = *reinterpret_cast<const uint16_t*>(blk + 208);
    }
    const int xch = M * (Q6XP / 16);
    for (int j = 0; j * 64 < xch; ++j) {
      const int id = min(j * 64 + lane, xch - 1);
      const int m = id / (Q6XP / 16), pos = min(id % (Q6XP / 16), cnt * 16 - 1);
      __builtin_amdgcn_global_load_lds((kq_gptr_t)(x + (int64_t)m * K + (int64_t)c0 * 256 + 16 * pos),
                                       (kq_lptr_t)(xw + j * 1024), 16, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
#pragma unroll
    for (int i = 0; i < Q6CH; ++i) {
      if (i < cnt) {
        const float d = h2f((uint16_t)q6_pull(dw[i], 4 * lj));  // column lj's d (lane 4 lj loaded it)
        // exact integer sums of this lane's 4 sub-blocks of the super-block:
        // |sc * S| < 128 * 16 * 127 * 32 < 2^23 per term
        int T[MB][4];
#pragma unroll
        for (int t = 0; t < MB; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) T[t][r] = 0;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          // ql bytes 64 hf + 16 h .. +15 (piece h of half hf) and qh bytes
          // 32 hf + 16 (h & 1) .. +15 (qh piece 2 hf + (h & 1)) of row lj
          const uint4 qlv = hf ? qlp[i][1] : qlp[i][0];
          uint32_t ql[4], qh[4];
          ql[0] = q6_pull(qlv.x, 4 * lj + h); ql[1] = q6_pull(qlv.y, 4 * lj + h);
          ql[2] = q6_pull(qlv.z, 4 * lj + h); ql[3] = q6_pull(qlv.w, 4 * lj + h);
          const int sq = 4 * lj + 2 * hf + (h & 1);
          qh[0] = q6_pull(qhp[i].x, sq); qh[1] = q6_pull(qhp[i].y, sq);
          qh[2] = q6_pull(qhp[i].z, sq); qh[3] = q6_pull(qhp[i].w, sq);
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) {
            const int qd = (h >> 1) + 2 * nb;  // quadrant of this lane's k-slots
            v4i bop;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t q = ((ql[e] >> (4 * nb)) & 0x0F0F0F0Fu) | (((qh[e] >> (2 * qd)) & 0x03030303u) << 4);
              const uint32_t tq = q ^ 0x20202020u;             // q - 32 as 6-bit two's complement
              bop[e] = (int)(tq | ((tq & 0x20202020u) * 6u));  // sign-extended to 8 bits
            }
            // scale of this lane's C-row group g = h: index 8 hf + 4 nb + h,
            // byte h of scale dword 2 hf + nb of column lj
            const uint32_t sw = q6_pull(scw[i], 4 * lj + 2 * hf + nb);
            const int sc = (int)(int8_t)((sw >> (8 * h)) & 0xFF);
#pragma unroll
            for (int t = 0; t < MB; ++t) {
              const int4 xv = *reinterpret_cast<const int4*>(xrow[t] + i * 256 + 128 * hf + 64 * nb + 16 * gA);
              const v4i aop = {xv.x, xv.y, xv.z, xv.w};
              const v4i cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop, bop, v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
              for (int r = 0; r < 4; ++r) T[t][r] += __mul24(sc, cc[r]);
            }
          }
        }
#pragma unroll
        for (int t = 0; t < MB; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) f[t][r] += d * (float)T[t][r];
      }
    }
    __builtin_amdgcn_wave_barrier();  // the next chunk's copies overwrite xw
  };

  const int sb0 = (wave * nsb) / Q6W, sb1 = ((wave + 1) * nsb) / Q6W;
  if (sb1 - sb0 <= Q6CH) {
    if (sb1 > sb0) chunk(sb0, sb1 - sb0);
  } else {
    for (int c0 = sb0; c0 < sb1; c0 += Q6CH) chunk(c0, min(Q6CH, sb1 - c0));
  }
  // C rows 4 g + r (g = lane / 16): sum the 4 sub-block groups, then the waves in fixed order
#pragma unroll
  for (int t = 0; t < MB; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      f[t][r] += __shfl_xor(f[t][r], 16, 64);
      f[t][r] += __shfl_xor(f[t][r], 32, 64);
    }
  if (wave > 0 && lane < 16) {
#pragma unroll
    for (int t = 0; t < MB; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) red6[wave - 1][t][lane][r] = f[t][r];
  }
  __syncthreads();
  if (wave == 0 && lane < 16) {
#pragma unroll
    for (int t = 0; t < MB; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = f[t][r];
#pragma unroll
        for (int wv = 0; wv < Q6W - 1; ++wv) v += red6[wv][t][lane][r];
        const int m = 4 * t + r, gn = n0 + lane;
        if (m < M && gn < N) st_out<OUT_DT>(out, (int64_t)m * N + gn, v * x_scale[m]);
      }
  }
}

void launch_gemv_q6k_mfma(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                          int M, int N, int K, hipStream_t st) {
  const dim3 grid((unsigned)((N + 15) / 16));
  const size_t lds = (size_t)Q6W * ((((size_t)M * Q6XP + 1023) & ~(size_t)1023) + Q6XP);
#define SL8_Q6M(MB)                                                                                   \
  switch (odt) {                                                                                      \
    case SL8_DTYPE_F16: gemv_q6k_mfma_kernel<SL8_DTYPE_F16, MB><<<grid, 64 * Q6W, lds, st>>>(x, xs, w, out, M, N, K); break; \
    case SL8_DTYPE_BF16: gemv_q6k_mfma_kernel<SL8_DTYPE_BF16, MB><<<grid, 64 * Q6W, lds, st>>>(x, xs, w, out, M, N, K); break; \
    default: gemv_q6k_mfma_kernel<SL8_DTYPE_F32, MB><<<grid, 64 * Q6W, lds, st>>>(x, xs, w, out, M, N, K); break; \
  }
  if (M <= 4) { SL8_Q6M(1) } else if (M <= 8) { SL8_Q6M(2) } else { SL8_Q6M(4) }
#undef SL8_Q6M
}

// smallest M on the int8 MFMA GEMVs (below: the VALU kernels). Config 4's
// shape, same box: M = 2 Q5_K 19.7 -> 17.0 us, Q6_K 29.4 -> 22.5 us; at M = 1
// the VALU kernels stay ahead (Q6_K 21.2 against 21.7 us)
#ifndef SL8_Q5_MFMA_MIN
#define SL8_Q5_MFMA_MIN 2
#endif
#ifndef SL8_Q6_MFMA_MIN
#define SL8_Q6_MFMA_MIN 2
#endif
#ifndef SL8_Q5_SMALL
#define SL8_Q5_SMALL 1
#endif
template <int FMT>
void launch_gemv_kq(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                    int M, int N, int K, hipStream_t st) {
  if (M >= (FMT == 6 ? SL8_Q6_MFMA_MIN : SL8_Q5_MFMA_MIN)) {  // the int8 MFMA GEMVs (Q5_K: the Q4_K kernel of gemm_q4k.hip)
    if (FMT == 5) launch_gemv_q5k_mfma(x, xs, w, out, odt, M, N, K, st);
    else launch_gemv_q6k_mfma(x, xs, w, out, odt, M, N, K, st);
    return;
  }
  if (FMT == 5 && SL8_Q5_SMALL) {  // Q5_K, M <= 2: the Q4_K M <= 2 kernel's layout (gemm_q4k.hip)
    launch_gemv_q5k_small(x, xs, w, out, odt, M, N, K, st);
    return;
  }
  if (M == 1) launch_gemv_kq_m<FMT, 1>(x, xs, w, out, odt, M, N, K, st);
  else launch_gemv_kq_m<FMT, 2>(x, xs, w, out, odt, M, N, K, st);
}

template <int FMT>
void launch_kq_tile(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                    int M, int N, int K, hipStream_t st) {
  // one workgroup per 128 x 128 tile; when the last round of tiles would hold
  // at most half the CUs, those tiles run as 4 row quarters each (a second
  // launch), which shortens that round (same per-element arithmetic)
  const int ntx = (N + KBN - 1) / KBN, T = ntx * ((M + KBM - 1) / KBM), P = cu_count();
  const int rem = T % P, nfull = (T >= P && rem > 0 && rem <= P / 2) ? T - rem : T;
  // XCD-aware tile order (kq_tile_coords) when the column tiles split evenly over the 8 XCDs
  const int xm = (SL8_KQ_XCD && ntx % 8 == 0) ? (M + KBM - 1) / KBM : 0;
#define SL8_KQT(KERN, RB, NW, G, T0)                                                               \
  switch (odt) {                                                                                   \
    case SL8_DTYPE_F16: KERN<SL8_DTYPE_F16, RB, NW><<<G, 64 * NW, 0, st>>>(x, xs, w, out, M, N, K, ntx, xm, T0); break; \
    case SL8_DTYPE_BF16: KERN<SL8_DTYPE_BF16, RB, NW><<<G, 64 * NW, 0, st>>>(x, xs, w, out, M, N, K, ntx, xm, T0); break; \
    default: KERN<SL8_DTYPE_F32, RB, NW><<<G, 64 * NW, 0, st>>>(x, xs, w, out, M, N, K, ntx, xm, T0); break;        \
  }
  if (FMT == 5) {
    if (SL8_KQ_NW8) { SL8_KQT(gemm_q5k_tile_kernel, 2, 8, nfull, 0) } else { SL8_KQT(gemm_q5k_tile_kernel, 4, 4, nfull, 0) }
    if (nfull < T) SL8_KQT(gemm_q5k_tile_kernel, 1, 4, 4 * (T - nfull), nfull)
  } else {
    if (SL8_Q6_NW8) { SL8_KQT(gemm_q6k_tile_kernel, 2, 8, nfull, 0) } else { SL8_KQT(gemm_q6k_tile_kernel, 4, 4, nfull, 0) }
    if (nfull < T) SL8_KQT(gemm_q6k_tile_kernel, 1, 4, 4 * (T - nfull), nfull)
  }
#undef SL8_KQT
}

int check_kq(const char* name, const int8_t* x, const float* xs, const uint8_t* w, void* out,
             int odt, int64_t M, int64_t N, int64_t K) {
  SL8_CHECK_ARG(odt == SL8_DTYPE_F16 || odt == SL8_DTYPE_BF16 || odt == SL8_DTYPE_F32,
                "out_dtype must be float16 or bfloat16 (or float32)");
  SL8_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "%s: bad shape", name);
  SL8_CHECK_ARG(K % 256 == 0, "%s needs K%%256==0, got %lld", name, (long long)K);
  SL8_CHECK_ARG(K <= 65536, "%s: K=%lld exceeds 65536", name, (long long)K);
  SL8_CHECK_ARG(N < (1LL << 31) && M < (1LL << 31), "%s: shape too large", name);
  if (M == 0 || N == 0 || K == 0) return SL8_OK;
  SL8_CHECK_ARG(x && xs && w && out, "%s: null pointer", name);
  SL8_CHECK_ARG(aligned(x, 16), "x must be 16-byte aligned for the vectorized int4 loads");
  SL8_CHECK_ARG(aligned(w, 16), "%s: weight must be 16-byte aligned", name);
  SL8_CHECK_ARG((M + KBM - 1) / KBM * ((N + KBN - 1) / KBN) < (1LL << 28), "%s: M*N too large", name);
  return SL8_OK;
}

}  // namespace
}  // namespace sl8

using namespace sl8;

extern "C" int sl8_gemm_q5k(const int8_t* x, const float* x_scale, const uint8_t* w, void* out,
                            int out_dtype, int64_t M, int64_t N, int64_t K, void* stream) {
  clear_error();
  int rc = check_kq("gemm_q5k", x, x_scale, w, out, out_dtype, M, N, K);
  if (rc != SL8_OK || M == 0 || N == 0 || K == 0) return rc;
  if (M <= 16) launch_gemv_kq<5>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K,
                                 static_cast<hipStream_t>(stream));
  else launch_kq_tile<5>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K,
                    static_cast<hipStream_t>(stream));
  SL8_CHECK_LAUNCH("gemm_q5k");
  return SL8_OK;
}

extern "C" int sl8_gemm_q6k(const int8_t* x, const float* x_scale, const uint8_t* w, void* out,
                            int out_dtype, int64_t M, int64_t N, int64_t K, void* stream) {
  clear_error();
  int rc = check_kq("gemm_q6k", x, x_scale, w, out, out_dtype, M, N, K);
  if (rc != SL8_OK || M == 0 || N == 0 || K == 0) return rc;
  if (M <= 16) launch_gemv_kq<6>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K,
                                 static_cast<hipStream_t>(stream));
  else launch_kq_tile<6>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K,
                    static_cast<hipStream_t>(stream));
  SL8_CHECK_LAUNCH("gemm_q6k");
  return SL8_OK;
}

extern "C" int sl8_gemm_decode_q5k(const int8_t* x, const float* x_scale, const uint8_t* w,
                                   void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                                   void* stream) {
  clear_error();
  int rc = check_kq("gemm_decode_q5k", x, x_scale, w, out, out_dtype, M, N, K);
  if (rc != SL8_OK || M == 0 || N == 0 || K == 0) return rc;
  SL8_CHECK_ARG(M <= 16, "gemm_decode_q5k supports M<=16, got M=%lld -- use the tile gemm_q5k for prefill",
                (long long)M);
  launch_gemv_kq<5>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K,
                    static_cast<hipStream_t>(stream));
  SL8_CHECK_LAUNCH("gemm_decode_q5k");
  return SL8_OK;
}

extern "C" int sl8_gemm_decode_q6k(const int8_t* x, const float* x_scale, const uint8_t* w,
                                   void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                                   void* stream) {
  clear_error();
  int rc = check_kq("gemm_decode_q6k", x, x_scale, w, out, out_dtype, M, N, K);
  if (rc != SL8_OK || M == 0 || N == 0 || K == 0) return rc;
  SL8_CHECK_ARG(M <= 16, "gemm_decode_q6k supports M<=16, got M=%lld -- use the tile gemm_q6k for prefill",
                (long long)M);
  launch_gemv_kq<6>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K,
                    static_cast<hipStream_t>(stream));
  SL8_CHECK_LAUNCH("gemm_decode_q6k");
  return SL8_OK;
}

extern "C" int sl8_dequant_q5k(const uint8_t* w, float* out, int64_t N, int64_t K, void* stream) {
  clear_error();
  SL8_CHECK_ARG(N >= 0 && K >= 0 && K % 256 == 0, "dequant_q5k needs K%%256==0, got %lld", (long long)K);
  if (N == 0 || K == 0) return SL8_OK;
  SL8_CHECK_ARG(w && out && aligned(w, 4), "dequant_q5k: null or misaligned pointer");
  const int64_t total = N * (K / 32);
  dequant_q5k_kernel<<<(unsigned)((total + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      w, out, N, (int)K);
  SL8_CHECK_LAUNCH("dequant_q5k");
  return SL8_OK;
}

extern "C" int sl8_dequant_q6k(const uint8_t* w, float* out, int64_t N, int64_t K, void* stream) {
  clear_error();
  SL8_CHECK_ARG(N >= 0 && K >= 0 && K % 256 == 0, "dequant_q6k needs K%%256==0, got %lld", (long long)K);
  if (N == 0 || K == 0) return SL8_OK;
  SL8_CHECK_ARG(w && out, "dequant_q6k: null pointer");
  const int64_t total = N * (K / 16);
  dequant_q6k_kernel<<<(unsigned)((total + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      w, out, N, (int)K);
  SL8_CHECK_LAUNCH("dequant_q6k");
  return SL8_OK;
}
