// Q4_K GEMV (M <= 16 activation rows) over native GGUF super-blocks, gfx950.
//
// Math (reference csrc/include/gemm_decode_dp4a.cuh:476-537 and
// csrc/include/gemm_q4k_dp4a.cuh:35-51):
//   y[m,n] = x_scale[m] * sum_j ( d*sc_j*<x_j, q_j> - dmin*m_j*sum(x_j) )
// over 32-element sub-blocks j; q in [0,15]; sc_j, m_j 6-bit.
//
// MI355X design. The weight stream (144 B per 256 weights) is the only HBM
// traffic that matters, so every weight byte is loaded once with 16-byte
// loads and unpacked in registers. The integer dot products run on the int8
// MFMA (v_mfma_i32_16x16x64_i8) instead of VALU dot4: one 16x16x64 MFMA
// covers one 32-byte nibble group (two sub-blocks, 64 weights) of 16 weight
// rows against up to 8 activation rows. The trick that keeps the two
// sub-blocks' sums apart inside one MFMA: A-operand rows 0..7 carry x for
// the low-nibble sub-block (zeros for the high half of k) and rows 8..15 the
// high-nibble sub-block, so C[i][n] is <x_m, q> of sub-block 2g + i/8.
//   A (16 x 64, "x"):  row i = (m = i%8, parity p = i/8)
//   B (64 x 16, "w"):  column n = weight row, k = the group's 64 nibbles
// k-slot mapping (lane group h = lane/16, byte b): h=0,1 -> low nibble of
// group byte 16h+b; h=2,3 -> high nibble of byte 16(h-2)+b. A and B use the
// same mapping, which is all the contraction needs.
// Per-sub-block affine scales are then applied in the integer domain:
//   T += sc_j * S_j (v_mad_i32_i24), U += m_j * xsum_j, and once per
//   super-block f += d*T - dmin*U (fp32). |T| < 2^24, so this is exact until
//   the final fp32 accumulate.
// Workgroup: 4 waves, 16 weight rows; the waves split the super-blocks of K
// and reduce through LDS in a fixed order (deterministic output).

#include "common.hpp"

namespace sl8 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int Q4K_BYTES = 144;
constexpr int GEMV_THREADS = 256;
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

template <int OUT_DT, int MT>
__global__ void __launch_bounds__(GEMV_THREADS)
gemv_q4k_kernel(const int8_t* __restrict__ x, const float* __restrict__ x_scale,
                const uint8_t* __restrict__ w, void* __restrict__ out, int M, int N, int K) {
  extern __shared__ int xs_lds[];  // [K/32][XS_MPAD] sub-block sums of x
  __shared__ float red[MT][4][64][4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nsub = K >> 5;
  const int nsb = K >> 8;

  // ---- x sub-block sums (rows >= M are zero) ----
  for (int idx = tid; idx < nsub * XS_MPAD; idx += GEMV_THREADS) {
    const int j = idx / XS_MPAD, m = idx % XS_MPAD;
    int s = 0;
    if (m < M) {
      const int4* p = reinterpret_cast<const int4*>(x + (int64_t)m * K + 32 * j);
      const int4 a = p[0], b = p[1];
      s = __builtin_amdgcn_sdot4(a.x, 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(a.y, 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(a.z, 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(a.w, 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(b.x, 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(b.y, 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(b.z, 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(b.w, 0x01010101, s, false);
    }
    xs_lds[idx] = s;
  }
  __syncthreads();

  const int lj = lane & 15;  // B column (weight row) / A row
  const int h = lane >> 4;   // k-slot group
  const int hp = h >> 1;     // nibble half this lane's B slots / C rows belong to
  const int n = blockIdx.x * GEMV_ROWS + lj;
  const bool n_ok = n < N;
  const uint8_t* wrow = w + (int64_t)(n_ok ? n : 0) * nsb * Q4K_BYTES;

  // A-operand row of this lane: m = mt*8 + (lj & 7), active iff parity matches.
  const int a_m = lj & 7;
  const bool a_on = ((lj >> 3) == hp);

  float f[MT][4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) f[t][r] = 0.f;

  const int sb0 = (wave * nsb) / 4, sb1 = ((wave + 1) * nsb) / 4;
  for (int sb = sb0; sb < sb1; ++sb) {
    const uint8_t* blk = wrow + (int64_t)sb * Q4K_BYTES;
    const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
    uint4 qv[4];
#pragma unroll
    for (int g = 0; g < 4; ++g)
      qv[g] = *reinterpret_cast<const uint4*>(blk + 16 + 32 * g + 16 * (h & 1));
    const ScMin sm = unpack_scmin(hdr.y, hdr.z, hdr.w);
    const float d = h2f(hdr.x & 0xFFFFu);
    const float dmin = h2f(hdr.x >> 16);

    int T[MT][4], U[MT][4];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) { T[t][r] = 0; U[t][r] = 0; }

#pragma unroll
    for (int g = 0; g < 4; ++g) {
      v4i bop;
      if (hp == 0) {
        bop.x = qv[g].x & 0x0F0F0F0F; bop.y = qv[g].y & 0x0F0F0F0F;
        bop.z = qv[g].z & 0x0F0F0F0F; bop.w = qv[g].w & 0x0F0F0F0F;
      } else {
        bop.x = (qv[g].x >> 4) & 0x0F0F0F0F; bop.y = (qv[g].y >> 4) & 0x0F0F0F0F;
        bop.z = (qv[g].z >> 4) & 0x0F0F0F0F; bop.w = (qv[g].w >> 4) & 0x0F0F0F0F;
      }
      const int j = 2 * g + hp;  // sub-block of this lane's C rows
      const int sc = byte_of(j < 4 ? sm.sc_lo : sm.sc_hi, j & 3);
      const int mn = byte_of(j < 4 ? sm.mn_lo : sm.mn_hi, j & 3);
      const int jg = sb * 8 + j;  // global sub-block index
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        v4i aop = {0, 0, 0, 0};
        const int am = t * 8 + a_m;
        if (a_on && am < M)
          aop = *reinterpret_cast<const v4i*>(x + (int64_t)am * K + sb * 256 + 64 * g + 16 * h);
        v4i c = {0, 0, 0, 0};
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop, bop, c, 0, 0, 0);
        const int4 xs4 = *reinterpret_cast<const int4*>(&xs_lds[jg * XS_MPAD + t * 8 + 4 * (h & 1)]);
        T[t][0] += __mul24(sc, c.x); T[t][1] += __mul24(sc, c.y);
        T[t][2] += __mul24(sc, c.z); T[t][3] += __mul24(sc, c.w);
        U[t][0] += __mul24(mn, xs4.x); U[t][1] += __mul24(mn, xs4.y);
        U[t][2] += __mul24(mn, xs4.z); U[t][3] += __mul24(mn, xs4.w);
      }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) f[t][r] += d * (float)T[t][r] - dmin * (float)U[t][r];
  }

#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[t][wave][lane][r] = f[t][r];
  __syncthreads();

  // One thread per output (m, n): fixed-order sum over waves and nibble halves.
  if (tid < MT * 8 * GEMV_ROWS) {
    const int mloc = tid / GEMV_ROWS, col = tid % GEMV_ROWS;
    const int t = mloc >> 3, mm = mloc & 7;
    const int gn = blockIdx.x * GEMV_ROWS + col;
    if (mloc < M && gn < N) {
      const int r = mm & 3, hl = mm >> 2;
      float s = 0.f;
#pragma unroll
      for (int wv = 0; wv < 4; ++wv)
#pragma unroll
        for (int p = 0; p < 2; ++p) s += red[t][wv][((p << 1) | hl) * 16 + col][r];
      st_out<OUT_DT>(out, (int64_t)mloc * N + gn, s * x_scale[mloc]);
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

template <int MT>
void launch_gemv_mt(const int8_t* x, const float* xs, const uint8_t* w, void* out, int odt,
                    int M, int N, int K, hipStream_t st) {
  const dim3 grid((unsigned)((N + GEMV_ROWS - 1) / GEMV_ROWS));
  const size_t lds = (size_t)(K / 32) * XS_MPAD * sizeof(int);
  switch (odt) {
    case SL8_DTYPE_F16:
      gemv_q4k_kernel<SL8_DTYPE_F16, MT><<<grid, GEMV_THREADS, lds, st>>>(x, xs, w, out, M, N, K);
      break;
    case SL8_DTYPE_BF16:
      gemv_q4k_kernel<SL8_DTYPE_BF16, MT><<<grid, GEMV_THREADS, lds, st>>>(x, xs, w, out, M, N, K);
      break;
    default:
      gemv_q4k_kernel<SL8_DTYPE_F32, MT><<<grid, GEMV_THREADS, lds, st>>>(x, xs, w, out, M, N, K);
      break;
  }
}

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

// LDS budget for the x sub-block sums: K/32 * 16 ints.
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
