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

#include "common.hpp"

namespace sl8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int Q4K_BYTES = 144;
constexpr int GEMV_ROWS = 16;
constexpr int XS_MPAD = 16;  // xsum LDS row pitch (activation rows)

// Packed 6-bit sub-scales / mins of one super-block (4 per dword, byte j%4).
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
__device__ __forceinline__ int byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFF; }

// Work split: a workgroup = GTILES 16-row MFMA tiles = 4 waves, each wave
// taking one quarter of the super-blocks of K; partial sums are reduced
// through LDS in a fixed order. Each wave issues every weight load of its
// share (up to GCH super-blocks per tile) before it waits for any of them,
// so a wave costs one memory round trip; meanwhile the workgroup stages the
// activations (M x K int8) into LDS, where the x operands are read from.
// At the config shape (N = 17408, K = 5120) this is 4352 waves at 4 waves
// per SIMD.
// Per group and row tile: one MFMA for <x, q> (scaled by sc_j in the integer
// domain with v_mad_i32_i24) and one MFMA whose B operand holds m_j in every
// slot of the sub-block, so it accumulates m_j * sum(x_j) over the
// super-block in its own accumulator.
constexpr int GCH = 5;     // super-blocks per wave and chunk
constexpr int GWAVES = 4;  // K split
constexpr int GTILES = 1;  // 16-row tiles per wave
constexpr int XLDS_MAX = 48 * 1024;

template <int OUT_DT, int MT, bool XLDS>
__global__ void __launch_bounds__(64 * GWAVES)
gemv_q4k_kernel(const int8_t* __restrict__ x, const float* __restrict__ x_scale,
                const uint8_t* __restrict__ w, void* __restrict__ out, int M, int N, int K) {
  __shared__ float red[GWAVES - 1][GTILES][MT][32][4];
  extern __shared__ __attribute__((aligned(16))) int8_t x_lds[];  // XLDS: x [M][K]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nsb = K >> 8;
  const int lj = lane & 15;  // B column (weight row in the tile) / A row
  const int h = lane >> 4;   // k-slot group: bytes 8h..8h+7 of each 32-byte nibble group
  const int hp = h >> 1;     // sub-block parity of this lane's C rows
  const int n0 = blockIdx.x * (GEMV_ROWS * GTILES);
  const int64_t row_bytes = (int64_t)nsb * Q4K_BYTES;
  const uint8_t* wrow[GTILES];
#pragma unroll
  for (int rt = 0; rt < GTILES; ++rt)
    wrow[rt] = w + (int64_t)min(n0 + rt * GEMV_ROWS + lj, N - 1) * row_bytes;
  const int a_m = lj & 7;    // A-operand row: activation t*8 + a_m, sub-block parity a_p
  const int a_p = lj >> 3;
  const uint32_t mlo = a_p == 0 ? 0xFFFFFFFFu : 0u, mhi = ~mlo;
  bool a_on[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) a_on[t] = t * 8 + a_m < M;
  const int sh = 8 * hp;     // byte of the lane's sub-block inside a scale dword pair

  float f[GTILES][MT][4];
#pragma unroll
  for (int rt = 0; rt < GTILES; ++rt)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) f[rt][t][r] = 0.f;

  const int sb0 = (wave * nsb) / GWAVES, sb1 = ((wave + 1) * nsb) / GWAVES;  // may be empty
  // the same chunk count for every wave keeps the staging barrier uniform
  const int nch = ((nsb + GWAVES - 1) / GWAVES + GCH - 1) / GCH;
  for (int c = 0; c < nch; ++c) {
    const int c0 = sb0 + c * GCH;
    uint4 hdr[GCH][GTILES];
    uint2 qv[GCH][GTILES][4];
#pragma unroll
    for (int i = 0; i < GCH; ++i) {
      const int sb = min(c0 + i, nsb - 1);  // always a valid block; unused ones are skipped
#pragma unroll
      for (int rt = 0; rt < GTILES; ++rt) {
        const uint8_t* blk = wrow[rt] + (int64_t)sb * Q4K_BYTES;
        hdr[i][rt] = *reinterpret_cast<const uint4*>(blk);
#pragma unroll
        for (int g = 0; g < 4; ++g)
          qv[i][rt][g] = *reinterpret_cast<const uint2*>(blk + 16 + 32 * g + 8 * h);
      }
    }
    if (XLDS && c == 0) {
      // activations into LDS while the first weight loads are in flight
      const int n16 = M * K / 16;
      for (int v = tid; v < n16; v += 64 * GWAVES)
        reinterpret_cast<int4*>(x_lds)[v] = reinterpret_cast<const int4*>(x)[v];
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < GCH; ++i) {
      if (c0 + i < sb1) {
        const int sb = c0 + i;
        ScMin sm[GTILES];
        int T[GTILES][MT][4];
        v4i U[GTILES][MT];
#pragma unroll
        for (int rt = 0; rt < GTILES; ++rt) {
          sm[rt] = unpack_scmin(hdr[i][rt].y, hdr[i][rt].z, hdr[i][rt].w);
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            U[rt][t] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int r = 0; r < 4; ++r) T[rt][t][r] = 0;
          }
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          v4i aop[MT];
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            const int64_t xo = (int64_t)min(t * 8 + a_m, M - 1) * K + sb * 256 + 64 * g + 32 * a_p + 8 * h;
            const uint2 xv = XLDS ? *reinterpret_cast<const uint2*>(x_lds + xo)
                                  : *reinterpret_cast<const uint2*>(x + xo);
            const uint32_t xlo = a_on[t] ? xv.x : 0u, xhi = a_on[t] ? xv.y : 0u;
            aop[t] = v4i{(int)(xlo & mlo), (int)(xhi & mlo), (int)(xlo & mhi), (int)(xhi & mhi)};
          }
#pragma unroll
          for (int rt = 0; rt < GTILES; ++rt) {
            const uint32_t w0 = qv[i][rt][g].x, w1 = qv[i][rt][g].y;
            const v4i bop = {(int)(w0 & 0x0F0F0F0Fu), (int)(w1 & 0x0F0F0F0Fu),
                             (int)((w0 >> 4) & 0x0F0F0F0Fu), (int)((w1 >> 4) & 0x0F0F0F0Fu)};
            // sub-blocks 2g (low slots) and 2g+1 (high slots) of this column's row
            const uint32_t scw = g < 2 ? sm[rt].sc_lo : sm[rt].sc_hi;
            const uint32_t mnw = g < 2 ? sm[rt].mn_lo : sm[rt].mn_hi;
            const int sc = (scw >> (16 * (g & 1) + sh)) & 0xFF;
            const uint32_t m_lo = ((mnw >> (16 * (g & 1))) & 0xFF) * 0x01010101u;
            const uint32_t m_hi = ((mnw >> (16 * (g & 1) + 8)) & 0xFF) * 0x01010101u;
            const v4i bmin = {(int)m_lo, (int)m_lo, (int)m_hi, (int)m_hi};
#pragma unroll
            for (int t = 0; t < MT; ++t) {
              const v4i z = {0, 0, 0, 0};
              const v4i cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop[t], bop, z, 0, 0, 0);
              U[rt][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop[t], bmin, U[rt][t], 0, 0, 0);
#pragma unroll
              for (int r = 0; r < 4; ++r) T[rt][t][r] += __mul24(sc, cc[r]);
            }
          }
        }
#pragma unroll
        for (int rt = 0; rt < GTILES; ++rt) {
          const float d = h2f(hdr[i][rt].x & 0xFFFFu);
          const float dmin = h2f(hdr[i][rt].x >> 16);
#pragma unroll
          for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              f[rt][t][r] += d * (float)T[rt][t][r] - dmin * (float)U[rt][t][r];
        }
      }
    }
  }

  // C row i = 4h + r holds activation row t*8 + (i & 7) of sub-block parity i >> 3:
  // add the two parities (lanes h and h^2), then the K quarters, in fixed order.
#pragma unroll
  for (int rt = 0; rt < GTILES; ++rt)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) f[rt][t][r] += __shfl_xor(f[rt][t][r], 32, 64);
  if (wave > 0 && lane < 32) {
#pragma unroll
    for (int rt = 0; rt < GTILES; ++rt)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave - 1][rt][t][lane][r] = f[rt][t][r];
  }
  __syncthreads();
  if (wave == 0 && lane < 32) {
#pragma unroll
    for (int rt = 0; rt < GTILES; ++rt)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = f[rt][t][r];
#pragma unroll
          for (int wv = 0; wv < GWAVES - 1; ++wv) v += red[wv][rt][t][lane][r];
          const int m = t * 8 + 4 * (h & 1) + r, gn = n0 + rt * GEMV_ROWS + lj;
          if (m < M && gn < N) st_out<OUT_DT>(out, (int64_t)m * N + gn, v * x_scale[m]);
        }
  }
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

template <int MT, bool XLDS>
void launch_gemv_mtx(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                     int M, int N, int K, hipStream_t st) {
  const dim3 grid((unsigned)((N + GEMV_ROWS * GTILES - 1) / (GEMV_ROWS * GTILES)));
  const size_t lds = XLDS ? (size_t)M * K : 0;
  switch (odt) {
    case SL8_DTYPE_F16:
      gemv_q4k_kernel<SL8_DTYPE_F16, MT, XLDS><<<grid, 64 * GWAVES, lds, st>>>(x, xs, w, out, M, N, K);
      break;
    case SL8_DTYPE_BF16:
      gemv_q4k_kernel<SL8_DTYPE_BF16, MT, XLDS><<<grid, 64 * GWAVES, lds, st>>>(x, xs, w, out, M, N, K);
      break;
    default:
      gemv_q4k_kernel<SL8_DTYPE_F32, MT, XLDS><<<grid, 64 * GWAVES, lds, st>>>(x, xs, w, out, M, N, K);
      break;
  }
}

// x goes to LDS when it is small (the decode shapes); otherwise operands are
// read from global memory (L2-resident).
template <int MT>
void launch_gemv_mt(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                    int M, int N, int K, hipStream_t st) {
  if ((int64_t)M * K <= XLDS_MAX) launch_gemv_mtx<MT, true>(x, xs, w, out, odt, M, N, K, st);
  else launch_gemv_mtx<MT, false>(x, xs, w, out, odt, M, N, K, st);
}

}  // namespace
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
  if (M <= 8) launch_gemv_mt<1>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K, st);
  else launch_gemv_mt<2>(x, x_scale, w, out, out_dtype, (int)M, (int)N, (int)K, st);
  SL8_CHECK_LAUNCH("gemm_decode_q4k");
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
  // 16-row activation slabs through the same MFMA kernel.
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
