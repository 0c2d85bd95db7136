// Q4_K GEMV (M <= 16 activation rows) over native GGUF super-blocks, gfx950.
//
// Math (reference csrc/include/gemm_decode_dp4a.cuh:476-537 and
// csrc/include/gemm_q4k_dp4a.cuh:35-51):
//   y[m,n] = x_scale[m] * sum_j ( d*sc_j*<x_j, q_j> - dmin*m_j*sum(x_j) )
// over 32-element sub-blocks j; q in [0,15]; sc_j, m_j 6-bit.
//
// MI355X design. The weight stream (144 B per 256 weights) is the only HBM
// traffic that matters, so every weight byte is loaded once (each lane owns
// distinct bytes) and unpacked in registers; a wave issues all loads of a
// chunk of super-blocks before consuming any of them. The integer dot products run on the int8
// MFMA (v_mfma_i32_16x16x64_i8) instead of VALU dot4: one 16x16x64 MFMA
// covers one 32-byte nibble group (two sub-blocks, 64 weights) of 16 weight
// rows against up to 8 activation rows. The trick that keeps the two
// sub-blocks' sums apart inside one MFMA: A-operand rows 0..7 carry x for
// the low-nibble sub-block (zeros for the high half of k) and rows 8..15 the
// high-nibble sub-block, so C[i][n] is <x_m, q> of sub-block 2g + i/8.
//   A (16 x 64, "x"):  row i = (m = i%8, parity p = i/8)
//   B (64 x 16, "w"):  column n = weight row, k = the group's 64 nibbles
// k-slot mapping (lane group h = lane/16, slot b = 0..15): slot b < 8 is the
// low nibble of group byte 8h+b, slot b >= 8 the high nibble of byte 8h+b-8;
// so a lane unpacks one 8-byte load into its 16 slots. A and B use the same
// mapping, which is all the contraction needs.
// Per-sub-block affine scales are then applied in the integer domain:
//   T += sc_j * S_j (v_mad_i32_i24), U += m_j * xsum_j, and once per
//   super-block f += d*T - dmin*U (fp32). |T| < 2^24, so this is exact until
//   the final fp32 accumulate.
// Workgroup: 4 waves, 16 weight rows; the waves split the super-blocks of K
// and reduce through LDS in a fixed order (deterministic output). The x
// sub-block sums each wave needs are formed in its own LDS slice.

#include "kquant.hpp"

namespace sl8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int Q4K_BYTES = 144;
constexpr int GEMV_ROWS = 16;
constexpr int XS_MPAD = 16;  // xsum LDS row pitch (activation rows)


// Work split: a workgroup = one 16-row MFMA tile = 4 waves, each wave taking
// one quarter of the super-blocks of K (in chunks of up to GCH); partial
// sums are reduced through LDS in a fixed order.
// Loads: for a coalesced stream, lane 4*r + c reads 16-byte piece c of weight
// row r (64 contiguous bytes per row and instruction) -- the MFMA operand
// layout wants lane r + 16*c instead, so after the loads land the pieces are
// moved across lanes with ds_bpermute (no LDS memory traffic). Every load of
// a chunk is issued before any is consumed (one round trip per chunk); the
// activation slice is copied into the wave's LDS area meanwhile.
// Operand mapping (lane = column lj + 16*h): lane h holds bytes 16h..16h+15
// of each 64-byte half L of the row's nibble array, i.e. elements
// 16(h&1)..+15 of sub-block 4L + 2(h>>1) (low nibbles) or 4L + 2(h>>1) + 1
// (high nibbles). A-operand rows 0..7 are activation rows for lane groups
// h = 0,1 (zero in groups 2,3), rows 8..15 the same activations for groups
// 2,3: C row 4h'+r then holds the sum over exactly one sub-block. Each
// (half, nibble) pair is one MFMA for <x, q> (scaled by sc_j in the integer
// domain with v_mad_i32_i24) plus one MFMA whose B operand holds m_j in
// every slot, accumulating m_j * sum(x_j) per super-block.
#ifndef SL8_GEMV_XBLDS
#define SL8_GEMV_XBLDS 1
#endif
// SL8_GEMV_FULLC: the K = 5 * GCH * GWAVES decode shapes take the straight-line
// path with a compile-time chunk count (see the dispatch at the end).
// SL8_GEMV_XFIRST: at MT = 1 the activation copies are issued before the
// weight loads. Config 4's shape, same box: M = 8 17.5 -> 17.0 us, M = 8 with
// per-block x scales 17.9 -> 16.9 us, M = 16 33.5 -> 32.9 us, Q5_K M = 8 20.4 -> 20.0 us.
// SL8_GEMV_MT2OCC: waves per SIMD of the 9 <= M <= 16 kernels (MT = 2). Config
// 4's shape, M = 16, same box: 1 (the register budget then left them at 2-3)
// 32.8 us, 3 31.1 us (per-block x scales 32.5 -> 30.7, Q5_K 38.5 -> 37.0), 4
// 31.0 us but 44.6 with per-block scales (spills).
#ifndef SL8_GEMV_MT2OCC
#define SL8_GEMV_MT2OCC 3
#endif
#ifndef SL8_GEMV_FULLC
#define SL8_GEMV_FULLC 1
#endif
#ifndef SL8_GEMV_XFIRST
#define SL8_GEMV_XFIRST 1
#endif
constexpr int GCH = 5;     // super-blocks per wave and chunk
constexpr int GWAVES = 4;  // K split
constexpr int GXPITCH = GCH * 256;  // LDS bytes per activation row and wave

typedef __attribute__((address_space(1))) const void* q4_gptr_t;
typedef __attribute__((address_space(3))) void* q4_lptr_t;


__device__ __forceinline__ uint32_t lane_pull(uint32_t v, int src_lane) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src_lane << 2, (int)v);
}

// MT = 1: at most 96 registers, so 5 waves per SIMD and every workgroup of
// the decode shapes (N / 16 = 1088 at N = 17408) is resident at once.
// FMT = 5: the same kernel on Q5_K super-blocks (176 bytes: header, 32 bytes of
// 5th bits qh, then the Q4_K-style nibbles): byte l of qh holds bit j for
// element l of sub-block j, so the operand lane of elements 16(h&1)..+15
// pulls qh bytes 16(h&1)..+15 of its row and the B operand is the code
// q = n + 16 b <= 31 (exact in int8); scales and mins as Q4_K.
// TPW = 16-row weight tiles per workgroup. The launcher uses 1: with 2 (each
// wave loads both tiles' weights before its single wait, the activation slice
// is staged once per 32 rows and the whole grid is resident at once) config 4
// at M = 8 measured 19.9 us against 17.3 us -- every wave then loads and
// computes in the same phase, so no compute overlaps the memory stream. XB: the
// activations carry one scale per 256-element block (x_scale [M, K/256],
// applied per super-block) instead of one per row; at M <= 8 those scales are
// copied into LDS with the activations (XBL) and the kernel keeps 5 waves per
// SIMD, at M > 8 they are held in registers.
// OPL: the weights are loaded straight into the MFMA operand layout (lane
// (row lj, group h) reads its own 16-byte pieces and the row's whole header)
// instead of the coalesced layout plus ds_bpermute moves. Same bytes, more
// cache-line segments per load instruction and no cross-lane moves; measured
// at config 4's shape: M = 4 15.9 -> 14.9 us, M = 16 36.2 -> 33.4 us, but
// M = 8 17.6 -> 18.1 us (its header registers spill at 5 waves per SIMD), so
// the launcher uses it for M <= 4 and M > 8.
template <int OUT_DT, int MT, int FMT = 4, int TPW = 1, bool XB = false, bool OPL = false>
__global__ void __launch_bounds__(64 * GWAVES, TPW == 2 ? 3 : (MT == 1 ? (FMT == 4 && (!XB || SL8_GEMV_XBLDS) ? 5 : 4) : SL8_GEMV_MT2OCC))
gemv_q4k_kernel(const int8_t* __restrict__ x, const float* __restrict__ x_scale,
                const uint8_t* __restrict__ w, void* __restrict__ out, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(16))) int8_t xl[];  // per wave: [M][GXPITCH]
  __shared__ float red[GWAVES - 1][TPW][MT][32][4];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nsb = K >> 8;
  const int lj = lane & 15;  // operand column (weight row in the tile) / A row
  const int h = lane >> 4;   // operand k-slot group
  const int hp = h >> 1;     // sub-block parity of this lane's k-slots and C rows
  const int lr = lane >> 2, lc = lane & 3;  // load role: weight row, 16-byte piece
  const int src_q = 4 * lj + h;             // lane holding (row lj, piece h)
  const int n0 = blockIdx.x * GEMV_ROWS * TPW;
  constexpr int BB = FMT == 4 ? Q4K_BYTES : 176;  // bytes per super-block
  constexpr int QS = FMT == 4 ? 16 : 48;          // offset of the nibbles
  const int64_t row_bytes = (int64_t)nsb * BB;
  const uint8_t* wrow[TPW];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt)
    wrow[tt] = w + (int64_t)min(n0 + GEMV_ROWS * tt + (OPL ? lj : lr), N - 1) * row_bytes;
  const int a_m = lj & 7;    // A-operand row: activation t*8 + a_m, parity lj >> 3
  const bool a_side = (lj >> 3) == hp;  // this lane's k-slots feed its A row
  bool a_on[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) a_on[t] = a_side && (t * 8 + a_m < M);
  // per wave: M activation rows rounded up to whole 1 KiB copies (a copy
  // writes 64 x 16 B, the last one past row M - 1), then one row of zeros
  // that the lanes whose A-operand row is unused read instead (no select
  // per operand)
  const int xarea = (M * GXPITCH + 1023) & ~1023;
  // XBL (XB, M <= 8): after the zero row, the chunk's per-block x scales [i][m],
  // read per super-block instead of held in 20 registers (which cost the
  // 5-wave occupancy): config 4 M = 8 18.1 -> 17.6 us (M = 16: 32.8 -> 33.7,
  // so not there)
  constexpr bool XBL = XB && SL8_GEMV_XBLDS && MT == 1;
  int8_t* xw = xl + (int64_t)wave * (xarea + GXPITCH + (XBL ? 256 : 0));
  int8_t* xz = xw + xarea;
  float* xsl = reinterpret_cast<float*>(xz + GXPITCH);
  for (int i = lane; i < GXPITCH / 16; i += 64) reinterpret_cast<uint4*>(xz)[i] = make_uint4(0, 0, 0, 0);

  float f[TPW][MT][4];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) f[tt][t][r] = 0.f;

  // One chunk of up to GCH super-blocks starting at c0.
  auto chunk = [&](const int c0, const int cnt) {
    // ---- activations of the chunk: M rows x cnt*256 bytes -> this wave's LDS area ----
    // (at MT = 1 issued before the weights, else after them)
    auto stage_x = [&]() {
      const int xch = M * (GXPITCH / 16);
      for (int j = 0; j * 64 < xch; ++j) {
        const int id = min(j * 64 + lane, xch - 1);
        const int m = id / (GXPITCH / 16), pos = min(id % (GXPITCH / 16), cnt * 16 - 1);
        __builtin_amdgcn_global_load_lds((q4_gptr_t)(x + (int64_t)m * K + (int64_t)c0 * 256 + 16 * pos),
                                         (q4_lptr_t)(xw + j * 1024), 16, 0, 0);
      }
      if constexpr (XBL) {
        // slot s = 8 i + m holds x_scale[m][c0 + i] (clamped: unused slots repeat)
        const int i = lane / 8, m = lane % 8;
        __builtin_amdgcn_global_load_lds(
            (q4_gptr_t)(x_scale + (int64_t)min(m, M - 1) * nsb + min(c0 + min(i, GCH - 1), nsb - 1)),
            (q4_lptr_t)xsl, 4, 0, 0);
      }
    };
    // ---- weights: header dword lc and two 16-byte nibble pieces per super-block ----
    uint32_t hd[TPW][GCH];
    uint4 qa[TPW][GCH], qb[TPW][GCH];
    uint2 qh8[TPW][FMT == 5 ? GCH : 1];  // Q5_K: qh bytes 8 lc .. 8 lc + 7 of the row
    uint4 hd4[TPW][OPL ? GCH : 1];       // OPL: the row's whole header
    uint4 qh16[TPW][OPL && FMT == 5 ? GCH : 1];  // OPL, Q5_K: qh bytes 16 (h & 1) .. +15
    constexpr bool XF = MT == 1 && TPW == 1 && !OPL && SL8_GEMV_XFIRST;
    if constexpr (XF) {
      stage_x();
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
      for (int i = 0; i < GCH; ++i) {
        const uint8_t* blk = wrow[tt] + (int64_t)min(c0 + i, nsb - 1) * BB;
        if constexpr (OPL) {
          // operand layout: lane (row lj, group h) loads its own pieces
          hd4[tt][i] = *reinterpret_cast<const uint4*>(blk);
          qa[tt][i] = *reinterpret_cast<const uint4*>(blk + QS + 16 * h);
          qb[tt][i] = *reinterpret_cast<const uint4*>(blk + QS + 64 + 16 * h);
          if constexpr (FMT == 5) qh16[tt][i] = *reinterpret_cast<const uint4*>(blk + 16 + 16 * (h & 1));
          continue;
        }
        hd[tt][i] = *reinterpret_cast<const uint32_t*>(blk + 4 * lc);
        qa[tt][i] = *reinterpret_cast<const uint4*>(blk + QS + 16 * lc);
        qb[tt][i] = *reinterpret_cast<const uint4*>(blk + QS + 64 + 16 * lc);
        if constexpr (FMT == 5) qh8[tt][i] = *reinterpret_cast<const uint2*>(blk + 16 + 8 * lc);
      }
    if constexpr (XF) __builtin_amdgcn_sched_barrier(0);
    else stage_x();
    // per-block activation scales of this lane's C rows (XB)
    float xsb[MT][4][XBL ? 1 : GCH];
    if constexpr (XB && !XBL) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = min(t * 8 + 4 * (h & 1) + r, M - 1);
#pragma unroll
          for (int i = 0; i < GCH; ++i) xsb[t][r][i] = x_scale[(int64_t)m * nsb + min(c0 + i, nsb - 1)];
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): weights and activations landed
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
    for (int i = 0; i < GCH; ++i) {
      if (i < cnt) {
        // ---- pieces to the operand layout ----
        uint32_t h0, h1, h2, h3;
        uint32_t qw[2][4];
        if constexpr (OPL) {
          h0 = hd4[tt][i].x; h1 = hd4[tt][i].y; h2 = hd4[tt][i].z; h3 = hd4[tt][i].w;
          qw[0][0] = qa[tt][i].x; qw[0][1] = qa[tt][i].y; qw[0][2] = qa[tt][i].z; qw[0][3] = qa[tt][i].w;
          qw[1][0] = qb[tt][i].x; qw[1][1] = qb[tt][i].y; qw[1][2] = qb[tt][i].z; qw[1][3] = qb[tt][i].w;
        } else {
          h0 = lane_pull(hd[tt][i], 4 * lj + 0); h1 = lane_pull(hd[tt][i], 4 * lj + 1);
          h2 = lane_pull(hd[tt][i], 4 * lj + 2); h3 = lane_pull(hd[tt][i], 4 * lj + 3);
          qw[0][0] = lane_pull(qa[tt][i].x, src_q); qw[0][1] = lane_pull(qa[tt][i].y, src_q);
          qw[0][2] = lane_pull(qa[tt][i].z, src_q); qw[0][3] = lane_pull(qa[tt][i].w, src_q);
          qw[1][0] = lane_pull(qb[tt][i].x, src_q); qw[1][1] = lane_pull(qb[tt][i].y, src_q);
          qw[1][2] = lane_pull(qb[tt][i].z, src_q); qw[1][3] = lane_pull(qb[tt][i].w, src_q);
        }
        const ScMin sm = unpack_scmin(h1, h2, h3);
        uint32_t qhw[4] = {0, 0, 0, 0};  // Q5_K: qh bytes 16(h&1) .. +15 of row lj
        if constexpr (OPL && FMT == 5) {
          qhw[0] = qh16[tt][i].x; qhw[1] = qh16[tt][i].y; qhw[2] = qh16[tt][i].z; qhw[3] = qh16[tt][i].w;
        } else if constexpr (FMT == 5) {
          const int s0 = 4 * lj + 2 * (h & 1);
          qhw[0] = lane_pull(qh8[tt][i].x, s0);
          qhw[1] = lane_pull(qh8[tt][i].y, s0);
          qhw[2] = lane_pull(qh8[tt][i].x, s0 + 1);
          qhw[3] = lane_pull(qh8[tt][i].y, s0 + 1);
        }
        int T[MT][4];
        v4i U[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          U[t] = v4i{0, 0, 0, 0};
#pragma unroll
          for (int r = 0; r < 4; ++r) T[t][r] = 0;
        }
#pragma unroll
        for (int L = 0; L < 2; ++L) {
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) {
            const int sh = 4 * nb;
            // sub-block 4L + 2hp + nb of this column's row
            const int sub = 4 * L + 2 * hp + nb;
            v4i bop;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              uint32_t c = (qw[L][e] >> sh) & 0x0F0F0F0Fu;
              if constexpr (FMT == 5) c |= ((qhw[e] >> sub) & 0x01010101u) << 4;
              bop[e] = (int)c;
            }
            const int bsel = 8 * (2 * hp + nb);
            const int sc = ((L == 0 ? sm.sc_lo : sm.sc_hi) >> bsel) & 0xFF;
            // byte (2hp + nb) of the packed mins in all four bytes (one v_perm
            // instead of a shift, a mask and a quarter-rate 32-bit multiply)
            const uint32_t mn = __builtin_amdgcn_perm(0u, L == 0 ? sm.mn_lo : sm.mn_hi,
                                                      (uint32_t)(2 * hp + nb) * 0x01010101u);
            const v4i bmin = {(int)mn, (int)mn, (int)mn, (int)mn};
#pragma unroll
            for (int t = 0; t < MT; ++t) {
              const int8_t* xrow = a_on[t] ? xw + (t * 8 + a_m) * GXPITCH : xz;
              const int4 xv = *reinterpret_cast<const int4*>(xrow + i * 256 + 32 * sub + 16 * (h & 1));
              const v4i aop = {xv.x, xv.y, xv.z, xv.w};
              const v4i z = {0, 0, 0, 0};
              const v4i cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop, bop, z, 0, 0, 0);
              U[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop, bmin, U[t], 0, 0, 0);
#pragma unroll
              for (int r = 0; r < 4; ++r) T[t][r] += __mul24(sc, cc[r]);
            }
          }
        }
        const float d = h2f(h0 & 0xFFFFu);
        const float dmin = h2f(h0 >> 16);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float part = d * (float)T[t][r] - dmin * (float)U[t][r];
            if constexpr (XBL) f[tt][t][r] += xsl[8 * i + 4 * (h & 1) + r] * part;
            else if constexpr (XB) f[tt][t][r] += xsb[t][r][i] * part;
            else f[tt][t][r] += part;
          }
      }
    }
    __builtin_amdgcn_wave_barrier();  // the next chunk's copies overwrite xw
  };

  const int sb0 = (wave * nsb) / GWAVES, sb1 = ((wave + 1) * nsb) / GWAVES;  // may be empty
  if (SL8_GEMV_FULLC && sb1 - sb0 == GCH) {
    // the decode shapes (K = 5120: 20 super-blocks, 5 per wave): one full
    // chunk with a compile-time count, so that no super-block's compute is
    // conditional -- with a run-time count the compiler sinks a conditional
    // block's weight loads into it, a second memory round trip per wave
    chunk(sb0, GCH);
  } else if (sb1 - sb0 <= GCH) {
    // one chunk, straight-line code (precise load waits)
    if (sb1 > sb0) chunk(sb0, sb1 - sb0);
  } else {
    for (int c0 = sb0; c0 < sb1; c0 += GCH) chunk(c0, min(GCH, sb1 - c0));
  }

  // C row i = 4h + r holds activation row t*8 + (i & 7) of sub-block parity i >> 3:
  // add the two parities (lanes h and h^2), then the K quarters, in fixed order.
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) f[tt][t][r] += __shfl_xor(f[tt][t][r], 32, 64);
  if (wave > 0 && lane < 32) {
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave - 1][tt][t][lane][r] = f[tt][t][r];
  }
  __syncthreads();
  if (wave == 0 && lane < 32) {
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = f[tt][t][r];
#pragma unroll
          for (int wv = 0; wv < GWAVES - 1; ++wv) v += red[wv][tt][t][lane][r];
          const int m = t * 8 + 4 * (h & 1) + r, gn = n0 + GEMV_ROWS * tt + lj;
          if (m < M && gn < N) st_out<OUT_DT>(out, (int64_t)m * N + gn, XB ? v : v * x_scale[m]);
        }
  }
}

// ---------------------------------------------------------------------------
// M <= 2: 16 weight rows per workgroup like the kernel above, with K split
// over SWAVES = 10 waves of up to SCH = 2 super-blocks (a fifth of the
// per-wave work of a 4-way split: the compute left after the last loads land
// is short, and at 64 VGPRs 8 waves share each SIMD), and the dot products run on VALU
// v_dot4 in the load layout itself -- lane 4r + c owns 16-byte piece c of
// each 64-byte half of weight row r, i.e. elements 16(c&1)..+15 of
// sub-blocks j = 2(c>>1) (low nibbles) and j+1 (high nibbles) of that half
// -- so nothing moves across lanes except the row's header dwords (a DPP
// quad broadcast). Activations are loaded first, then every weight load of
// the chunk; the activations go to LDS (with their 16-element sums, shared
// by all rows) as soon as they land, and super-block i is computed as soon
// as its own loads land while later ones are still in flight.
// ---------------------------------------------------------------------------
template <int R>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, R * 0x55, 0xF, 0xF, false);
}

#ifndef SL8_GEMV_SWAVES
#define SL8_GEMV_SWAVES 10
#endif
#ifndef SL8_GEMV_SCH
#define SL8_GEMV_SCH 2
#endif
constexpr int SWAVES = SL8_GEMV_SWAVES;  // K split of the M <= 2 kernel
constexpr int SCH = SL8_GEMV_SCH;        // its super-blocks per wave and chunk
constexpr int SXPITCH = SCH * 256;
// M = 1: at most 64 VGPRs, so 8 waves per SIMD and nearly the whole decode
// grid (1088 workgroups x 10 waves at N = 17408) is resident at once
#ifndef SL8_GEMV_SOCC
#define SL8_GEMV_SOCC 8
#endif
#ifndef SL8_GEMV_SOCC5
#define SL8_GEMV_SOCC5 6
#endif
// FMT = 5: Q5_K super-blocks (176 bytes: header, 32 bytes of 5th bits qh, then
// the Q4_K nibble layout); lane (r, c) also loads qh bytes 16 (c & 1) .. +15,
// the 5th bits of its elements (byte l holds bit j for element l of
// sub-block j), and each code is n + 16 b.
template <int OUT_DT, int MR, bool XB = false, int FMT = 4>
__global__ void __launch_bounds__(64 * SWAVES, (SL8_GEMV_SOCC > 0 && MR == 1) ? (FMT == 4 ? SL8_GEMV_SOCC : SL8_GEMV_SOCC5) : 1)
gemv_q4k_small_kernel(const int8_t* __restrict__ x, const float* __restrict__ x_scale,
                      const uint8_t* __restrict__ w, void* __restrict__ out, int M, int N, int K) {
  constexpr int XC = (MR * SXPITCH + 1023) / 1024;  // 16-byte activation pieces per lane
  __shared__ __attribute__((aligned(16))) int8_t xs_l[SWAVES][XC * 1024];
  __shared__ __attribute__((aligned(16))) int xsum_l[SWAVES][MR][SCH][2][8];  // [m][i][half][j]
  __shared__ float red[SWAVES - 1][16][MR];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nsb = K >> 8;
  const int r = lane >> 2, c = lane & 3;
  const int g = c >> 1, half = c & 1;
  const int n0 = blockIdx.x * GEMV_ROWS;
  constexpr int BB = FMT == 4 ? Q4K_BYTES : 176;  // bytes per super-block
  constexpr int QS = FMT == 4 ? 16 : 48;          // offset of the nibbles
  const int64_t row_bytes = (int64_t)nsb * BB;
  const uint8_t* wrow = w + (int64_t)min(n0 + r, N - 1) * row_bytes;
  int8_t* xw = &xs_l[wave][0];

  float f[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) f[m] = 0.f;

  auto chunk = [&](const int c0, const int cnt) {
    // ---- activations first: M rows x cnt*256 bytes, lane-linear 16-byte pieces ----
    const int xch = M * (SXPITCH / 16);
    static_assert(XC <= 3, "activation pieces per lane");
    auto xload = [&](int j) -> uint4 {
      const int id = min(j * 64 + lane, xch - 1);
      const int m = id / (SXPITCH / 16), pos = min(id % (SXPITCH / 16), cnt * 16 - 1);
      return *reinterpret_cast<const uint4*>(x + (int64_t)m * K + (int64_t)c0 * 256 + 16 * pos);
    };
    const uint4 xq0 = xload(0);
    const uint4 xq1 = XC > 1 ? xload(1) : xq0;
    const uint4 xq2 = XC > 2 ? xload(2) : xq0;
    __builtin_amdgcn_sched_barrier(0);
    // ---- then every weight load of the chunk ----
    // (two per-lane base pointers plus immediate offsets; a partial chunk
    // re-reads its last super-block instead of running past the row)
    uint32_t hd[SCH];
    uint4 qa[SCH], qb[SCH];
    const uint8_t* bh = wrow + (int64_t)c0 * BB + 4 * c;
    const uint8_t* bq = wrow + (int64_t)c0 * BB + 16 * c;
    uint4 qh5[FMT == 5 ? SCH : 1];  // Q5_K: qh bytes 16 half .. +15
#pragma unroll
    for (int i = 0; i < SCH; ++i) {
      const int ii = cnt == SCH ? i : min(i, cnt - 1);
      hd[i] = *reinterpret_cast<const uint32_t*>(bh + ii * BB);
      qa[i] = *reinterpret_cast<const uint4*>(bq + ii * BB + QS);
      qb[i] = *reinterpret_cast<const uint4*>(bq + ii * BB + QS + 64);
      if constexpr (FMT == 5)
        qh5[i] = *reinterpret_cast<const uint4*>(wrow + (int64_t)(c0 + ii) * BB + 16 + 16 * half);
    }
    __builtin_amdgcn_sched_barrier(0);
    // ---- activations to LDS ([m][SXPITCH]) and their 16-element sums ----
    *reinterpret_cast<uint4*>(xw + 16 * lane) = xq0;
    if (XC > 1) *reinterpret_cast<uint4*>(xw + 1024 + 16 * lane) = xq1;
    if (XC > 2) *reinterpret_cast<uint4*>(xw + 2048 + 16 * lane) = xq2;
    __builtin_amdgcn_wave_barrier();
    // sum over elements 16*half2..+15 of sub-block j2 of super-block i2, row m2
    for (int e = lane; e < MR * SCH * 16; e += 64) {
      const int m2 = e / (SCH * 16), i2 = (e / 16) % SCH, half2 = (e / 8) & 1, j2 = e & 7;
      const int4 v = *reinterpret_cast<const int4*>(xw + m2 * SXPITCH + i2 * 256 + 32 * j2 + 16 * half2);
      int sacc = __builtin_amdgcn_sdot4(v.x, 0x01010101, 0, false);
      sacc = __builtin_amdgcn_sdot4(v.y, 0x01010101, sacc, false);
      sacc = __builtin_amdgcn_sdot4(v.z, 0x01010101, sacc, false);
      sacc = __builtin_amdgcn_sdot4(v.w, 0x01010101, sacc, false);
      xsum_l[wave][m2][i2][half2][j2] = sacc;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < SCH; ++i) {
      if (i < cnt) {
        // header dwords of row r, from the quad's lanes 4r .. 4r+3
        const uint32_t h0 = quad_bcast<0>(hd[i]), h1 = quad_bcast<1>(hd[i]);
        const uint32_t h2 = quad_bcast<2>(hd[i]), h3 = quad_bcast<3>(hd[i]);
        const ScMin sm = unpack_scmin(h1, h2, h3);
        // this lane's sub-blocks: j0 = 2g, j0+1 (half 0 of the row), j0+4, j0+5 (half 1)
        const int bs = 16 * g;
        const int sc0 = (sm.sc_lo >> bs) & 0xFF, sc1 = (sm.sc_lo >> (bs + 8)) & 0xFF;
        const int sc4 = (sm.sc_hi >> bs) & 0xFF, sc5 = (sm.sc_hi >> (bs + 8)) & 0xFF;
        const int mn0 = (sm.mn_lo >> bs) & 0xFF, mn1 = (sm.mn_lo >> (bs + 8)) & 0xFF;
        const int mn4 = (sm.mn_hi >> bs) & 0xFF, mn5 = (sm.mn_hi >> (bs + 8)) & 0xFF;
        const uint32_t wa[4] = {qa[i].x, qa[i].y, qa[i].z, qa[i].w};
        const uint32_t wbq[4] = {qb[i].x, qb[i].y, qb[i].z, qb[i].w};
        const float d = h2f(h0 & 0xFFFFu), dmin = h2f(h0 >> 16);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const int8_t* xb = xw + m * SXPITCH + i * 256 + 16 * half;
          const int4 x0 = *reinterpret_cast<const int4*>(xb + 32 * (2 * g));
          const int4 x1 = *reinterpret_cast<const int4*>(xb + 32 * (2 * g + 1));
          const int4 x4 = *reinterpret_cast<const int4*>(xb + 32 * (2 * g + 4));
          const int4 x5 = *reinterpret_cast<const int4*>(xb + 32 * (2 * g + 5));
          const int xa0[4] = {x0.x, x0.y, x0.z, x0.w}, xa1[4] = {x1.x, x1.y, x1.z, x1.w};
          const int xa4[4] = {x4.x, x4.y, x4.z, x4.w}, xa5[4] = {x5.x, x5.y, x5.z, x5.w};
          int p0 = 0, p1 = 0, p4 = 0, p5 = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            if constexpr (FMT == 4) {
              p0 = __builtin_amdgcn_sdot4(xa0[k], (int)(wa[k] & 0x0F0F0F0Fu), p0, false);
              p1 = __builtin_amdgcn_sdot4(xa1[k], (int)((wa[k] >> 4) & 0x0F0F0F0Fu), p1, false);
              p4 = __builtin_amdgcn_sdot4(xa4[k], (int)(wbq[k] & 0x0F0F0F0Fu), p4, false);
              p5 = __builtin_amdgcn_sdot4(xa5[k], (int)((wbq[k] >> 4) & 0x0F0F0F0Fu), p5, false);
            } else {
              // codes n + 16 b of sub-blocks 2g, 2g+1 (qa) and 2g+4, 2g+5 (qb):
              // bit j of each qh byte goes to bit 4 of the code of sub-block j
              const uint32_t hk = k == 0 ? qh5[i].x : k == 1 ? qh5[i].y : k == 2 ? qh5[i].z : qh5[i].w;
              const uint32_t q0 = (wa[k] & 0x0F0F0F0Fu) | (((hk >> (2 * g)) & 0x01010101u) << 4);
              const uint32_t q1 = ((wa[k] >> 4) & 0x0F0F0F0Fu) | (((hk >> (2 * g + 1)) & 0x01010101u) << 4);
              const uint32_t q4 = (wbq[k] & 0x0F0F0F0Fu) | (((hk >> (2 * g + 4)) & 0x01010101u) << 4);
              const uint32_t q5 = ((wbq[k] >> 4) & 0x0F0F0F0Fu) | (((hk >> (2 * g + 5)) & 0x01010101u) << 4);
              p0 = __builtin_amdgcn_sdot4(xa0[k], (int)q0, p0, false);
              p1 = __builtin_amdgcn_sdot4(xa1[k], (int)q1, p1, false);
              p4 = __builtin_amdgcn_sdot4(xa4[k], (int)q4, p4, false);
              p5 = __builtin_amdgcn_sdot4(xa5[k], (int)q5, p5, false);
            }
          }
          const int* xsr = &xsum_l[wave][m][i][half][0];
          const int2 s01 = *reinterpret_cast<const int2*>(xsr + 2 * g);
          const int2 s45 = *reinterpret_cast<const int2*>(xsr + 4 + 2 * g);
          const int T = __mul24(sc0, p0) + __mul24(sc1, p1) + __mul24(sc4, p4) + __mul24(sc5, p5);
          const int U = __mul24(mn0, s01.x) + __mul24(mn1, s01.y) + __mul24(mn4, s45.x) +
                        __mul24(mn5, s45.y);
          const float part = d * (float)T - dmin * (float)U;
          if constexpr (XB) f[m] += x_scale[(int64_t)m * nsb + c0 + i] * part;  // per-256-block scale
          else f[m] += part;
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // the next chunk rewrites xw / xsum_l
  };

  const int sb0 = (wave * nsb) / SWAVES, sb1 = ((wave + 1) * nsb) / SWAVES;  // may be empty
  if (sb1 - sb0 == SCH) {
    chunk(sb0, SCH);  // the decode shapes: one full chunk, immediate offsets
  } else {
    for (int c0 = sb0; c0 < sb1; c0 += SCH) chunk(c0, min(SCH, sb1 - c0));
  }

  // quad sum (the 4 pieces of a row), then the K quarters in fixed order
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    f[m] += __shfl_xor(f[m], 1, 64);
    f[m] += __shfl_xor(f[m], 2, 64);
  }
  if (wave > 0 && c == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m) red[wave - 1][r][m] = f[m];
  }
  __syncthreads();
  if (wave == 0 && c == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float v = f[m];
#pragma unroll
      for (int wv = 0; wv < SWAVES - 1; ++wv) v += red[wv][r][m];
      const int gn = n0 + r;
      if (m < M && gn < N) st_out<OUT_DT>(out, (int64_t)m * N + gn, XB ? v : v * x_scale[m]);
    }
  }
}

// ---------------------------------------------------------------------------
// Tiled Q4_K GEMM for M > 16 (prefill; reference csrc/include/gemm_q4k_dp4a.cuh:
// 60-199, csrc/kernel/gemm_dp4a.cu:146-193): a 128 x 128 output tile per
// workgroup of 8 waves, two per SIMD, each owning 32 output columns x 64 rows
// (2 blocks of 32 x 32; each B operand is built by the two waves of its
// columns: with 4 waves over all 128 rows, one per SIMD, a single wave's VALU
// issue rate bounded the kernel). Per super-block the
// x tile (128 x 256 int8) and the 128 weight super-blocks (144 B each) are
// copied global -> LDS one super-block ahead (double-buffered). The products
// stay exact integers on v_mfma_i32_32x32x32_i8, one MFMA per 32-element
// sub-block j (K = 32):
//   T_j = <x_j, q_j * sc_j> with the 6-bit sc_j split in 3-bit halves so each
//         B operand fits int8: q * (sc & 7) and q * (sc >> 3) (<= 105; one
//         32-bit multiply scales 4 nibbles at once, no carries), combined as
//         T_lo + 8 T_hi;
// and once per super-block f += d * (T_lo + 8 T_hi) (fp32). The min term
//   U = sum_j m_j * sum(x_j) is one v_mfma_f32_32x32x16_f16 per row block and
// super-block on the x half-sums and the mins (both exact in fp16; U is an
// exact fp32 integer), applied as f -= dmin * U one super-block later (the
// half-sums of the tile's rows are formed once, spread over the waves, and
// shared through LDS).
// x chunks are XOR-swizzled in LDS by row (rows are 256 B = one bank line);
// weight rows are 144 B apart, which already spreads 16 rows over all banks.
// ---------------------------------------------------------------------------
// SL8_KQ_NW8=0: the full tiles on 4 waves (one per SIMD, RB = 4)
#ifndef SL8_KQ_NW8
#define SL8_KQ_NW8 1
#endif
constexpr int TBM = 128, TBN = 128;  // output tile

template <int OUT_DT, int RB, int NW = 4>
__global__ void __launch_bounds__(64 * NW, 1)
gemm_q4k_tile_kernel(const int8_t* __restrict__ x, const float* __restrict__ x_scale,
                     const uint8_t* __restrict__ w, void* __restrict__ out, int M, int N, int K,
                     int nt_x, int xcd_m, int tile0) {
  // RB row blocks (32 rows) per wave, NW waves per workgroup: a full tile is
  // RB = 4, NW = 4 (one wave per SIMD, every wave over all 128 rows) or RB = 2,
  // NW = 8 (two waves per SIMD, each over 64 rows); RB = 1, NW = 4 is a row
  // quarter of a tile (the short last round)
  constexpr bool QTR = RB * NW < 16;
  constexpr int NT = 64 * NW;
  constexpr int WCH = (TBN * 9 + NT - 1) / NT * NT;  // weight-tile 16-B chunks, whole copies
  __shared__ __attribute__((aligned(16))) int8_t xs0[TBM * 256];
  __shared__ __attribute__((aligned(16))) int8_t xs1[TBM * 256];
  __shared__ __attribute__((aligned(16))) uint8_t ws0[WCH * 16];
  __shared__ __attribute__((aligned(16))) uint8_t ws1[WCH * 16];
  // full tiles: the fp16 A operands of the min-term MFMA (x half-sums) of one
  // super-block, [slot][row block][lane], formed by the waves together and
  // read after the next workgroup barrier
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
  const int n0 = ct * TBN, m0 = rt * TBM;
  const int rb0 = QTR ? (int)(blockIdx.x & 3) : 0;
  const int cg = wave & 3;                                  // the wave's 32 output columns
  const int rbw = QTR ? rb0 : (NW == 8 ? (wave >> 2) * RB : 0);  // its first row block
  const int nsb = K >> 8;
  const int64_t row_bytes = (int64_t)nsb * Q4K_BYTES;

  // copies of super-block sb into (xd, wd); chunk P of the tile lands at P*16
  auto load = [&](int sb, int8_t* xd, uint8_t* wd) __attribute__((always_inline)) {
    constexpr int XCH = QTR ? 512 : TBM * 16;  // a quarter copies only its 32 rows
#pragma unroll
    for (int i = 0; i < XCH / NT; ++i) {
      const int P0 = (QTR ? rb0 * 512 : 0) + i * NT;
      const int P = P0 + tid, row = P >> 4;
      const int c = (P & 15) ^ (row & 15);
      const int8_t* src = x + (int64_t)min(m0 + row, M - 1) * K + (int64_t)sb * 256 + 16 * c;
      __builtin_amdgcn_global_load_lds((q4_gptr_t)src, (q4_lptr_t)(xd + (P0 + wave * 64) * 16), 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < WCH / NT; ++i) {
      const int P = min(i * NT + tid, TBN * 9 - 1), row = P / 9, c = P - 9 * row;
      const uint8_t* src = w + (int64_t)min(n0 + row, N - 1) * row_bytes + (int64_t)sb * Q4K_BYTES + 16 * c;
      __builtin_amdgcn_global_load_lds((q4_gptr_t)src, (q4_lptr_t)(wd + (i * NT + wave * 64) * 16), 16, 0, 0);
    }
  };

  typedef int v16i_t __attribute__((ext_vector_type(16)));
  typedef float v16f_t __attribute__((ext_vector_type(16)));
  // wave (cg, row group) owns weight rows 32 cg .. 32 cg + 31 (output columns)
  // for the activation rows of its RB row blocks. K step j of a super-block is
  // sub-block j (lane half h holds its elements 16 h .. 16 h + 15); step j + 1's
  // A reads and B operands are formed while step j's MFMAs run (one
  // scheduling region per step).
  float f[RB][16];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int e = 0; e < 16; ++e) f[rb][e] = 0.f;

  // Min term U = sum_j m_j * xsum_j on one v_mfma_f32_32x32x16_f16 per row
  // block and super-block: A = the 16-element half-sums of x (k = 8 h + j,
  // |sum| <= 16 * 127 = 2032: exact in fp16), B = m_j (6-bit, exact) for both
  // halves, so U comes out as an exact fp32 integer (|U| <= 8 * 4064 * 63 <
  // 2^24). In a full tile the half-sums of the 4 row blocks are formed once
  // (NW = 4: wave w sums row block w; NW = 8: wave w row block w & 3, sub-blocks
  // 4 (w >> 2) .. +3) and published in LDS; every wave reads its row blocks'
  // after the next super-block's barrier, so U of super-block sb is formed
  // (and f -= dmin * U applied) one super-block late. Quarter waves share their
  // rows and form their operand themselves, and apply U just as late, so the
  // quarter launch's per-element arithmetic stays that of the full tiles.
  float u_dmin = 0.f;  // dmin of the super-block whose U is pending
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
    const uint8_t* wr = wt + (32 * cg + l32) * Q4K_BYTES;
    const uint4 hd = *reinterpret_cast<const uint4*>(wr);
    const float d = h2f(hd.x & 0xFFFFu), dmin = h2f(hd.x >> 16);
    const ScMin sm = unpack_scmin(hd.y, hd.z, hd.w);
    uint32_t qw[4][4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint4 qv = *reinterpret_cast<const uint4*>(wr + 16 + 32 * g + 16 * h);
      qw[g][0] = qv.x; qw[g][1] = qv.y; qw[g][2] = qv.z; qw[g][3] = qv.w;
    }
    float hsum[8];
    v4i A[2][RB], bl[2], bh[2];
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
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t nib = (qw[j >> 1][e] >> (4 * (j & 1))) & 0x0F0F0F0Fu;
        bl[buf][e] = (int)mul_bytes(nib, sc & 7);  // <= 15 * 7 per byte
        bh[buf][e] = (int)mul_bytes(nib, sc >> 3);
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
      }
      // the half-sums: a quarter wave sums step j's own A operand; in a full
      // tile this wave's JN sub-blocks are spread over the steps
      if constexpr (JN == 8) xsum_half(j);
      else if (j & 1) xsum_half(j >> 1);
      if (j < 7) build(j + 1, c ^ 1);
      __builtin_amdgcn_sched_group_barrier(0x100, RB + (QTR ? 0 : 1), 0);  // the LDS reads first
#pragma unroll
      for (int k = 0; k < 2 * RB; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, RB == 4 ? 4 : 8, 0);  // VALU
      }
    }
    // the min-term operands of this super-block
    v8h ub;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      ub[jj] = (_Float16)(float)(((jj < 4 ? sm.mn_lo : sm.mn_hi) >> (8 * (jj & 3))) & 0xFF);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int e = 0; e < 16; ++e) f[rb][e] += d * (float)(tl[rb][e] + (th[rb][e] << 3));
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
  // slot: the LDS slot this super-block's half-sums go to (full tiles); -2
  // for the first super-block (no U pending yet, slot 0)
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

void launch_gemm_tile(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                      int M, int N, int K, hipStream_t st) {
  // one workgroup per 128 x 128 tile; when the last round of tiles would hold
  // at most half the CUs, those tiles run as 4 row quarters each (a second
  // launch), which shortens that round (same per-element arithmetic)
  const int ntx = (N + TBN - 1) / TBN, T = ntx * ((M + TBM - 1) / TBM), P = cu_count();
  const int rem = T % P, nfull = (T >= P && rem > 0 && rem <= P / 2) ? T - rem : T;
  // XCD-aware tile order (kq_tile_coords) when the column tiles split evenly over the 8 XCDs
  const int xm = (SL8_KQ_XCD && ntx % 8 == 0) ? (M + TBM - 1) / TBM : 0;
#define SL8_Q4T(RB, NW, G, T0)                                                                              \
  switch (odt) {                                                                                            \
    case SL8_DTYPE_F16: gemm_q4k_tile_kernel<SL8_DTYPE_F16, RB, NW><<<G, 64 * NW, 0, st>>>(x, xs, w, out, M, N, K, ntx, xm, T0); break; \
    case SL8_DTYPE_BF16: gemm_q4k_tile_kernel<SL8_DTYPE_BF16, RB, NW><<<G, 64 * NW, 0, st>>>(x, xs, w, out, M, N, K, ntx, xm, T0); break; \
    default: gemm_q4k_tile_kernel<SL8_DTYPE_F32, RB, NW><<<G, 64 * NW, 0, st>>>(x, xs, w, out, M, N, K, ntx, xm, T0); break;        \
  }
  if (SL8_KQ_NW8) { SL8_Q4T(2, 8, nfull, 0) } else { SL8_Q4T(4, 4, nfull, 0) }
  if (nfull < T) SL8_Q4T(1, 4, 4 * (T - nfull), nfull)
#undef SL8_Q4T
}

__global__ void dequant_q4k_kernel(const uint8_t* __restrict__ w, float* __restrict__ out,
                                   int64_t N, int K) {
  // one thread per (row, sub-block): 32 outputs
  const int nsub = K >> 5, nsb = K >> 8;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N * nsub) return;
  const int64_t n = t / nsub;
  const int jg = (int)(t % nsub);
  const int sb = jg >> 3, j = jg & 7;
  const uint8_t* blk = w + (n * nsb + sb) * Q4K_BYTES;
  const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
  const ScMin sm = unpack_scmin(hdr.y, hdr.z, hdr.w);
  const int sc = byte_of(j < 4 ? sm.sc_lo : sm.sc_hi, j & 3);
  const int mn = byte_of(j < 4 ? sm.mn_lo : sm.mn_hi, j & 3);
  const float dsc = h2f(hdr.x & 0xFFFFu) * (float)sc;
  const float dm = h2f(hdr.x >> 16) * (float)mn;
  const uint8_t* qs = blk + 16 + 32 * (j >> 1);
  const int shift = (j & 1) ? 4 : 0;
  float* o = out + n * K + (int64_t)jg * 32;
  for (int e = 0; e < 32; ++e) o[e] = dsc * (float)((qs[e] >> shift) & 0xF) - dm;
}

template <int MR, bool XB = false, int FMT = 4>
void launch_gemv_small(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                       int M, int N, int K, hipStream_t st) {
  const dim3 grid((unsigned)((N + GEMV_ROWS - 1) / GEMV_ROWS));
  switch (odt) {
    case SL8_DTYPE_F16:
      gemv_q4k_small_kernel<SL8_DTYPE_F16, MR, XB, FMT><<<grid, 64 * SWAVES, 0, st>>>(x, xs, w, out, M, N, K);
      break;
    case SL8_DTYPE_BF16:
      gemv_q4k_small_kernel<SL8_DTYPE_BF16, MR, XB, FMT><<<grid, 64 * SWAVES, 0, st>>>(x, xs, w, out, M, N, K);
      break;
    default:
      gemv_q4k_small_kernel<SL8_DTYPE_F32, MR, XB, FMT><<<grid, 64 * SWAVES, 0, st>>>(x, xs, w, out, M, N, K);
      break;
  }
}

template <int MT, bool XB = false>
void launch_gemv_mt(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                    int M, int N, int K, hipStream_t st) {
  const dim3 grid((unsigned)((N + GEMV_ROWS - 1) / GEMV_ROWS));
  const size_t lds = (size_t)GWAVES * ((((size_t)M * GXPITCH + 1023) & ~(size_t)1023) + GXPITCH +
                                       (XB && SL8_GEMV_XBLDS && MT == 1 ? 256 : 0));
#define SL8_GM(DT, OP) gemv_q4k_kernel<DT, MT, 4, 1, XB, OP><<<grid, 64 * GWAVES, lds, st>>>(x, xs, w, out, M, N, K)
#define SL8_GM_DT(OP)                                   \
  switch (odt) {                                        \
    case SL8_DTYPE_F16: SL8_GM(SL8_DTYPE_F16, OP); break;   \
    case SL8_DTYPE_BF16: SL8_GM(SL8_DTYPE_BF16, OP); break; \
    default: SL8_GM(SL8_DTYPE_F32, OP); break;             \
  }
  if (MT == 2 || M <= 4) {
    SL8_GM_DT(true)
  } else {
    SL8_GM_DT(false)
  }
#undef SL8_GM_DT
#undef SL8_GM
}

}  // namespace

// Q5_K decode GEMV for M <= 2 on the M <= 2 kernel above (called from gemm_kq56.hip).
void launch_gemv_q5k_small(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                           int M, int N, int K, hipStream_t st) {
  if (M == 1) launch_gemv_small<1, false, 5>(x, xs, w, out, odt, M, N, K, st);
  else launch_gemv_small<2, false, 5>(x, xs, w, out, odt, M, N, K, st);
}

// operand-layout loads for Q5_K too at M <= 4 and 9 <= M <= 16 (config 4's
// shape: M = 4 18.9 -> 18.6 us, M = 16 40.8 -> 39.2 us; M = 8 unchanged)
#ifndef SL8_Q5_OPLM
#define SL8_Q5_OPLM 4
#endif
#ifndef SL8_Q5_OPL2
#define SL8_Q5_OPL2 1
#endif
// Q5_K decode GEMV (3 <= M <= 16) on the MFMA kernel above (called from gemm_kq56.hip).
void launch_gemv_q5k_mfma(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                          int M, int N, int K, hipStream_t st) {
  const dim3 grid((unsigned)((N + GEMV_ROWS - 1) / GEMV_ROWS));
  const size_t lds = (size_t)GWAVES * ((((size_t)M * GXPITCH + 1023) & ~(size_t)1023) + GXPITCH);
#define SL8_Q5M(MT, OP)                                                                               \
  switch (odt) {                                                                                      \
    case SL8_DTYPE_F16: gemv_q4k_kernel<SL8_DTYPE_F16, MT, 5, 1, false, OP><<<grid, 64 * GWAVES, lds, st>>>(x, xs, w, out, M, N, K); break; \
    case SL8_DTYPE_BF16: gemv_q4k_kernel<SL8_DTYPE_BF16, MT, 5, 1, false, OP><<<grid, 64 * GWAVES, lds, st>>>(x, xs, w, out, M, N, K); break; \
    default: gemv_q4k_kernel<SL8_DTYPE_F32, MT, 5, 1, false, OP><<<grid, 64 * GWAVES, lds, st>>>(x, xs, w, out, M, N, K); break; \
  }
  if (M <= SL8_Q5_OPLM) { SL8_Q5M(1, true) } else if (M <= 8) { SL8_Q5M(1, false) } else if (SL8_Q5_OPL2) { SL8_Q5M(2, true) } else { SL8_Q5M(2, false) }
#undef SL8_Q5M
}

}  // namespace sl8

namespace sl8 {
namespace {

int check_q4k(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
              int64_t M, int64_t N, int64_t K) {
  SL8_CHECK_ARG(odt == SL8_DTYPE_F16 || odt == SL8_DTYPE_BF16 || odt == SL8_DTYPE_F32,
                "out_dtype must be float16 or bfloat16 (or float32)");
  SL8_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "q4k: bad shape");
  SL8_CHECK_ARG(K % 256 == 0, "q4k needs K%%256==0, got %lld", (long long)K);
  SL8_CHECK_ARG(K <= (1 << 20), "q4k: K=%lld too large", (long long)K);
  if (M == 0 || N == 0 || K == 0) return SL8_OK;
  SL8_CHECK_ARG(x && xs && w && out, "q4k: null pointer");
  SL8_CHECK_ARG(aligned(x, 16), "x must be 16-byte aligned for the vectorized int4 loads");
  SL8_CHECK_ARG(aligned(w, 16), "q4k: weight must be 16-byte aligned");
  return SL8_OK;
}

}  // namespace
}  // namespace sl8

using namespace sl8;

// K bound keeping every integer partial sum well inside int32.
static constexpr int64_t kMaxGemvK = 65536;

extern "C" int sl8_gemm_decode_q4k(const int8_t* x, const float* x_scale, const uint8_t* w,
                                   void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                                   void* stream) {
  clear_error();
  int rc = check_q4k(x, x_scale, w, out, out_dtype, M, N, K);
  if (rc != SL8_OK || M == 0 || N == 0 || K == 0) return rc;
  SL8_CHECK_ARG(M <= 16, "gemm_decode_q4k supports M<=16, got M=%lld -- use the tile gemm_q4k for prefill",
                (long long)M);
  SL8_CHECK_ARG(K <= kMaxGemvK, "gemm_decode_q4k: K=%lld exceeds %lld", (long long)K,
                (long long)kMaxGemvK);
  SL8_CHECK_ARG(N < (1LL << 31), "gemm_decode_q4k: N too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (M == 1) launch_gemv_small<1>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K, st);
  else if (M == 2) launch_gemv_small<2>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K, st);
  else if (M <= 8) launch_gemv_mt<1>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K, st);
  else launch_gemv_mt<2>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K, st);
  SL8_CHECK_LAUNCH("gemm_decode_q4k");
  return SL8_OK;
}

// Decode GEMV with one activation scale per 256-element block (BASELINE
// config 4's activation format): x_scale [M, K/256] multiplies each
// super-block's exact integer sums instead of the row total.
extern "C" int sl8_gemm_decode_q4k_xblock(const int8_t* x, const float* x_scale, const uint8_t* w,
                                          void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                                          void* stream) {
  clear_error();
  int rc = check_q4k(x, x_scale, w, out, out_dtype, M, N, K);
  if (rc != SL8_OK || M == 0 || N == 0 || K == 0) return rc;
  SL8_CHECK_ARG(M <= 16, "gemm_decode_q4k supports M<=16, got M=%lld -- use the tile gemm_q4k for prefill",
                (long long)M);
  SL8_CHECK_ARG(K <= kMaxGemvK, "gemm_decode_q4k: K=%lld exceeds %lld", (long long)K,
                (long long)kMaxGemvK);
  SL8_CHECK_ARG(N < (1LL << 31), "gemm_decode_q4k: N too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (M == 1) launch_gemv_small<1, true>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K, st);
  else if (M == 2) launch_gemv_small<2, true>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K, st);
  else if (M <= 8) launch_gemv_mt<1, true>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K, st);
  else launch_gemv_mt<2, true>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K, st);
  SL8_CHECK_LAUNCH("gemm_decode_q4k_xblock");
  return SL8_OK;
}

extern "C" int sl8_gemm_q4k(const int8_t* x, const float* x_scale, const uint8_t* w, void* out,
                            int out_dtype, int64_t M, int64_t N, int64_t K, void* stream) {
  clear_error();
  int rc = check_q4k(x, x_scale, w, out, out_dtype, M, N, K);
  if (rc != SL8_OK || M == 0 || N == 0 || K == 0) return rc;
  SL8_CHECK_ARG(K <= kMaxGemvK, "gemm_q4k: K=%lld exceeds %lld", (long long)K, (long long)kMaxGemvK);
  SL8_CHECK_ARG(N < (1LL << 31), "gemm_q4k: N too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int esz = out_dtype == SL8_DTYPE_F32 ? 4 : 2;
  if (M > 16) {
    SL8_CHECK_ARG(M < (1LL << 31) && (M + TBM - 1) / TBM * ((N + TBN - 1) / TBN) < (1LL << 28), "gemm_q4k: M*N too large");
    launch_gemm_tile(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K, st);
    SL8_CHECK_LAUNCH("gemm_q4k");
    return SL8_OK;
  }
  // M <= 16: one 16-row activation slab through the GEMV MFMA kernel.
  for (int64_t m0 = 0; m0 < M; m0 += 16) {
    const int64_t mt = (M - m0) < 16 ? (M - m0) : 16;
    char* o = static_cast<char*>(out) + m0 * N * esz;
    if (mt <= 8) launch_gemv_mt<1>(x + m0 * K, x_scale + m0, w, o, out_dtype, (int)mt, (int)N, (int)K, st);
    else launch_gemv_mt<2>(x + m0 * K, x_scale + m0, w, o, out_dtype, (int)mt, (int)N, (int)K, st);
  }
  SL8_CHECK_LAUNCH("gemm_q4k");
  return SL8_OK;
}

extern "C" int sl8_dequant_q4k(const uint8_t* w, float* out, int64_t N, int64_t K, void* stream) {
  clear_error();
  SL8_CHECK_ARG(N >= 0 && K >= 0 && K % 256 == 0, "dequant_q4k needs K%%256==0, got %lld",
                (long long)K);
  if (N == 0 || K == 0) return SL8_OK;
  SL8_CHECK_ARG(w && out, "dequant_q4k: null pointer");
  SL8_CHECK_ARG(aligned(w, 16), "dequant_q4k: weight must be 16-byte aligned");
  const int64_t total = N * (K / 32);
  dequant_q4k_kernel<<<(unsigned)((total + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      w, out, N, (int)K);
  SL8_CHECK_LAUNCH("dequant_q4k");
  return SL8_OK;
}
