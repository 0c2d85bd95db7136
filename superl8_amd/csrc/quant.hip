// Per-row symmetric int8 quantisation and K-smoothing for gfx950.
//
// Numerics contract (reference csrc/include/quant_rowwise.cuh:33-91 and
// superl8/quant/core.py:47-62,70-95):
//   scale = amax|row| * fp32(1/127)   (reciprocal multiply, not division)
//   safe  = scale == 0 ? 1 : scale
//   q     = clamp(rint(x / safe), -127, 127)   with IEEE round-to-nearest
//           division and round-half-to-even.
// K-smoothing subtracts the fp32 per-channel key mean and rounds back to the
// storage dtype before quantising, exactly as torch.sub(k, mean, out=k_s).
//
// Layout: one row is handled by LPR lanes of a wave64 (LPR in {16,32,64});
// 256-thread blocks hold 256/LPR rows. Rows are read twice (amax pass, code
// pass); the second read is served by L2 for the row sizes used here.

#include "common.hpp"

#include <cmath>
#include <type_traits>
#include <string>

namespace sl8 {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}
void clear_error() { g_last_error.clear(); }

namespace {

constexpr int QTHREADS = 256;

// Reduction over aligned groups of LPR lanes (a power of two <= 64) with no
// LDS round trip: DPP inside a 16-lane row (quad_perm [1,0,3,2], quad_perm
// [2,3,0,1], row_half_mirror, row_mirror: after each step a lane holds the
// reduction over 2, 4, 8, 16 lanes), then v_permlane16_swap across the row
// pair and v_permlane32_swap across the wave halves. Every lane of the group
// ends with the result; op must be associative and commutative (max, integer
// add: exact in any order).
template <int LPR, typename F>
__device__ __forceinline__ uint32_t lane_group_reduce(uint32_t v, F op) {
  static_assert(LPR >= 1 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "LPR: a power of two <= 64");
  auto dpp = [](uint32_t x, auto ctrl) __attribute__((always_inline)) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, decltype(ctrl)::value, 0xF, 0xF, false);
  };
  if constexpr (LPR >= 2) v = op(v, dpp(v, std::integral_constant<int, 0xB1>{}));
  if constexpr (LPR >= 4) v = op(v, dpp(v, std::integral_constant<int, 0x4E>{}));
  if constexpr (LPR >= 8) v = op(v, dpp(v, std::integral_constant<int, 0x141>{}));
  if constexpr (LPR >= 16) v = op(v, dpp(v, std::integral_constant<int, 0x140>{}));
  if constexpr (LPR >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = op(r[0], r[1]);
  }
  if constexpr (LPR >= 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = op(r[0], r[1]);
  }
  return v;
}
// v >= 0 and not NaN (an amax started at 0 and grown by fmaxf, which drops
// NaN): the unsigned order of the bit patterns is the float order, and 0 is
// the identity of the unsigned max the DPP moves fold into
template <int LPR>
__device__ __forceinline__ float lane_group_max(float v) {
  return __uint_as_float(lane_group_reduce<LPR>(__float_as_uint(v), [](uint32_t a, uint32_t b) {
    return a > b ? a : b;
  }));
}
template <int LPR>
__device__ __forceinline__ int lane_group_sum(int v) {
  return (int)lane_group_reduce<LPR>((uint32_t)v, [](uint32_t a, uint32_t b) { return a + b; });
}

template <int DT> struct Elem;
template <> struct Elem<SL8_DTYPE_F16> {
  using T = uint16_t;
  __device__ static float ld(const T* p, int64_t i) { return h2f(p[i]); }
  __device__ static float round(float v) { return h2f(f2h_bits(v)); }
};
template <> struct Elem<SL8_DTYPE_BF16> {
  using T = uint16_t;
  __device__ static float ld(const T* p, int64_t i) { return bf2f(p[i]); }
  __device__ static float round(float v) { return bf2f(f2bf_bits(v)); }
};
template <> struct Elem<SL8_DTYPE_F32> {
  using T = float;
  __device__ static float ld(const T* p, int64_t i) { return p[i]; }
  __device__ static float round(float v) { return v; }
};

// Value of element d of a row after the optional mean shift.
template <int DT, bool MEAN>
__device__ __forceinline__ float row_val(const typename Elem<DT>::T* xr, const float* mr, int d) {
  float v = Elem<DT>::ld(xr, d);
  if constexpr (MEAN) v = Elem<DT>::round(v - mr[d]);
  return v;
}

__device__ __forceinline__ int8_t code_of(float v, float safe) {
  float r = rintf(__fdiv_rn(v, safe));
  r = fminf(fmaxf(r, -127.f), 127.f);
  return static_cast<int8_t>(r);
}

// rows = G*N; row r uses mean row r / rows_per_mean.
template <int DT, int LPR, bool MEAN>
__global__ void __launch_bounds__(QTHREADS)
quant_rows_kernel(const typename Elem<DT>::T* __restrict__ x, const float* __restrict__ mean,
                  int8_t* __restrict__ q, float* __restrict__ scale, int64_t rows,
                  int64_t rows_per_mean, int K, float scale_mul) {
  using T = typename Elem<DT>::T;
  const int lane = threadIdx.x % LPR;
  const int64_t row = (int64_t)blockIdx.x * (QTHREADS / LPR) + threadIdx.x / LPR;
  const bool live = row < rows;
  const int64_t r = live ? row : 0;
  const T* xr = x + r * K;
  const float* mr = MEAN ? mean + (r / rows_per_mean) * K : nullptr;

  float amax = 0.f;
  if (live) {
    for (int d = lane; d < K; d += LPR) amax = fmaxf(amax, fabsf(row_val<DT, MEAN>(xr, mr, d)));
  }
  amax = lane_group_max<LPR>(amax);
  if (!live) return;

  const float s = amax * (1.0f / 127.0f);
  const float safe = (s == 0.f) ? 1.f : s;
  if (lane == 0) scale[row] = safe * scale_mul;

  int8_t* qr = q + r * K;
  if ((K & 3) == 0) {
    // 4 codes per 32-bit store.
    for (int d = lane * 4; d < K; d += LPR * 4) {
      uint32_t packed = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        packed |= (uint32_t)(uint8_t)code_of(row_val<DT, MEAN>(xr, mr, d + e), safe) << (8 * e);
      *reinterpret_cast<uint32_t*>(qr + d) = packed;
    }
  } else {
    for (int d = lane; d < K; d += LPR) qr[d] = code_of(row_val<DT, MEAN>(xr, mr, d), safe);
  }
}


// Vectorised variant: LPR lanes per row (LPR = 256: one workgroup per row),
// each lane holding NV 16-byte vectors of the row in registers for both the
// amax and the code pass (one HBM read per element). Needs K a multiple of
// the elements per 16 bytes (EPV) and a 16-byte aligned base.
template <int DT> struct VecIO;
template <> struct VecIO<SL8_DTYPE_F16> {
  static constexpr int EPV = 8;
  __device__ static void unpack(uint4 v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) { f[2 * i] = h2f(w[i] & 0xFFFF); f[2 * i + 1] = h2f(w[i] >> 16); }
  }
};
template <> struct VecIO<SL8_DTYPE_BF16> {
  static constexpr int EPV = 8;
  __device__ static void unpack(uint4 v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) { f[2 * i] = bf2f(w[i] & 0xFFFF); f[2 * i + 1] = bf2f(w[i] >> 16); }
  }
};
template <> struct VecIO<SL8_DTYPE_F32> {
  static constexpr int EPV = 4;
  __device__ static void unpack(uint4 v, float* f) {
    f[0] = __uint_as_float(v.x); f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z); f[3] = __uint_as_float(v.w);
  }
};

template <int DT, int LPR, int NV, bool MEAN>
__global__ void __launch_bounds__(QTHREADS)
quant_rows_vec_kernel(const typename Elem<DT>::T* __restrict__ x, const float* __restrict__ mean,
                      int8_t* __restrict__ q, float* __restrict__ scale, int64_t rows,
                      int64_t rows_per_mean, int K, float scale_mul) {
  using T = typename Elem<DT>::T;
  constexpr int EPV = VecIO<DT>::EPV;
  const int lane = threadIdx.x % LPR;
  const int64_t row = (int64_t)blockIdx.x * (QTHREADS / LPR) + threadIdx.x / LPR;
  const bool live = row < rows;
  const int64_t r = live ? row : 0;
  const T* xr = x + r * K;
  const float* mr = MEAN ? mean + (r / rows_per_mean) * K : nullptr;
  const int nvec = K / EPV;

  float f[NV][EPV];
  float amax = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int vi = v * LPR + lane;
    const bool ok = live && vi < nvec;
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (ok) raw = reinterpret_cast<const uint4*>(xr)[vi];
    VecIO<DT>::unpack(raw, f[v]);
    if constexpr (MEAN) {
#pragma unroll
      for (int e = 0; e < EPV; ++e)
        f[v][e] = ok ? Elem<DT>::round(f[v][e] - mr[vi * EPV + e]) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < EPV; ++e) amax = fmaxf(amax, fabsf(f[v][e]));
  }
  if constexpr (LPR <= 64) {
    amax = lane_group_max<LPR>(amax);
  } else {
    __shared__ float red[QTHREADS / 64];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < QTHREADS / 64; ++w) amax = fmaxf(amax, red[w]);
  }
  if (!live) return;
  const float s = amax * (1.0f / 127.0f);
  const float safe = (s == 0.f) ? 1.f : s;
  if (lane == 0) scale[row] = safe * scale_mul;
  int8_t* qr = q + r * K;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int vi = v * LPR + lane;
    if (vi < nvec) {
      uint32_t w[EPV / 4];
#pragma unroll
      for (int i = 0; i < EPV / 4; ++i) {
        w[i] = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[i] |= (uint32_t)(uint8_t)code_of(f[v][4 * i + e], safe) << (8 * e);
      }
      if constexpr (EPV == 8) *reinterpret_cast<uint2*>(qr + vi * EPV) = make_uint2(w[0], w[1]);
      else *reinterpret_cast<uint32_t*>(qr + vi * EPV) = w[0];
    }
  }
}

template <int DT, bool MEAN>
int launch_quant(const void* x, const float* mean, int8_t* q, float* scale, int64_t rows,
                 int64_t rows_per_mean, int64_t K, float scale_mul, hipStream_t st) {
  using T = typename Elem<DT>::T;
  const T* xp = static_cast<const T*>(x);
  auto go = [&](auto lpr_tag) {
    constexpr int LPR = decltype(lpr_tag)::value;
    const int64_t rpb = QTHREADS / LPR;
    const dim3 grid((unsigned)((rows + rpb - 1) / rpb));
    quant_rows_kernel<DT, LPR, MEAN><<<grid, QTHREADS, 0, st>>>(xp, mean, q, scale, rows,
                                                                rows_per_mean, (int)K, scale_mul);
  };
  constexpr int EPV = VecIO<DT>::EPV;
  if (K % EPV == 0 && aligned(x, 16) && aligned(q, EPV) && K / EPV <= 8 * QTHREADS) {
    const int64_t nvec = K / EPV;
    auto gv = [&](auto lpr_tag, auto nv_tag) {
      constexpr int LPR = decltype(lpr_tag)::value, NV = decltype(nv_tag)::value;
      const int64_t rpb = QTHREADS / LPR;
      const dim3 grid((unsigned)((rows + rpb - 1) / rpb));
      quant_rows_vec_kernel<DT, LPR, NV, MEAN><<<grid, QTHREADS, 0, st>>>(
          xp, mean, q, scale, rows, rows_per_mean, (int)K, scale_mul);
    };
    using I = std::integral_constant<int, 1>;
    if (nvec <= 16) gv(std::integral_constant<int, 16>{}, I{});
    else if (nvec <= 32) gv(std::integral_constant<int, 32>{}, I{});
    else if (nvec <= 64) gv(std::integral_constant<int, 64>{}, I{});
    else if (nvec <= 128) gv(std::integral_constant<int, 64>{}, std::integral_constant<int, 2>{});
    else if (nvec <= 256) gv(std::integral_constant<int, 256>{}, I{});
    else if (nvec <= 512) gv(std::integral_constant<int, 256>{}, std::integral_constant<int, 2>{});
    else if (nvec <= 1024) gv(std::integral_constant<int, 256>{}, std::integral_constant<int, 4>{});
    else gv(std::integral_constant<int, 256>{}, std::integral_constant<int, 8>{});
  } else if (K <= 128) {
    go(std::integral_constant<int, 16>{});
  } else if (K <= 512) {
    go(std::integral_constant<int, 32>{});
  } else {
    go(std::integral_constant<int, 64>{});
  }
  SL8_CHECK_LAUNCH("quantize_i8_rowwise");
  return SL8_OK;
}

int dispatch_quant(const void* x, int dt, const float* mean, int8_t* q, float* scale,
                   int64_t rows, int64_t rows_per_mean, int64_t K, float scale_mul,
                   hipStream_t st) {
  if (mean) {
    switch (dt) {
      case SL8_DTYPE_F16: return launch_quant<SL8_DTYPE_F16, true>(x, mean, q, scale, rows, rows_per_mean, K, scale_mul, st);
      case SL8_DTYPE_BF16: return launch_quant<SL8_DTYPE_BF16, true>(x, mean, q, scale, rows, rows_per_mean, K, scale_mul, st);
      default: return launch_quant<SL8_DTYPE_F32, true>(x, mean, q, scale, rows, rows_per_mean, K, scale_mul, st);
    }
  }
  switch (dt) {
    case SL8_DTYPE_F16: return launch_quant<SL8_DTYPE_F16, false>(x, nullptr, q, scale, rows, 1, K, scale_mul, st);
    case SL8_DTYPE_BF16: return launch_quant<SL8_DTYPE_BF16, false>(x, nullptr, q, scale, rows, 1, K, scale_mul, st);
    default: return launch_quant<SL8_DTYPE_F32, false>(x, nullptr, q, scale, rows, 1, K, scale_mul, st);
  }
}

// ---- K mean -------------------------------------------------------------
// fp16: every value is an integer multiple of 2^-24 below 2^16 in magnitude,
// so sum(x * 2^24) is an exact int64 for N < 2^23 rows: the mean does not
// depend on summation order. Blocks take (64 columns, a chunk of rows); a
// block's exact partial sum is added to the int64 workspace with an integer
// atomic (exact, so still order free), and a last pass scales it.
constexpr int MEAN_COLS = 64;
constexpr int MEAN_PHASES = 16;
constexpr int MEAN_CHUNK = 256;  // rows per block

__global__ void __launch_bounds__(256) i64_zero_kernel(unsigned long long* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0ull;
}

__global__ void __launch_bounds__(MEAN_COLS * MEAN_PHASES)
k_mean_f16_kernel(const uint16_t* __restrict__ k, unsigned long long* __restrict__ acc, int64_t N,
                  int D) {
  __shared__ long long part[MEAN_PHASES][MEAN_COLS];
  const int col = threadIdx.x % MEAN_COLS;
  const int ph = threadIdx.x / MEAN_COLS;
  const int64_t g = blockIdx.y;
  const int d = blockIdx.x * MEAN_COLS + col;
  const int64_t n0 = (int64_t)blockIdx.z * MEAN_CHUNK;
  const int64_t n1 = min(N, n0 + MEAN_CHUNK);
  long long a = 0;
  if (d < D) {
    const uint16_t* kg = k + g * N * D + d;
#pragma unroll 4
    for (int64_t n = n0 + ph; n < n1; n += MEAN_PHASES)
      a += (long long)ldexpf(h2f(kg[n * D]), 24);  // exact: |v| * 2^24 < 2^40, integral
  }
  part[ph][col] = a;
  __syncthreads();
  if (ph == 0 && d < D) {
    long long t = 0;
#pragma unroll
    for (int p = 0; p < MEAN_PHASES; ++p) t += part[p][col];
    atomicAdd(acc + g * D + d, (unsigned long long)t);  // two's complement: exact mod 2^64
  }
}

__global__ void __launch_bounds__(256)
k_mean_finish_kernel(const unsigned long long* __restrict__ acc, float* __restrict__ mean,
                     int64_t n, int64_t N) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) mean[i] = (float)(((double)(long long)acc[i] * 0x1p-24) / (double)N);
}

// bf16 / f32: fp64 running sum over rows in index order (one thread per column).
template <int DT>
__global__ void __launch_bounds__(MEAN_COLS)
k_mean_seq_kernel(const typename Elem<DT>::T* __restrict__ k, float* __restrict__ mean,
                  int64_t N, int D) {
  const int64_t g = blockIdx.y;
  const int d = blockIdx.x * MEAN_COLS + threadIdx.x;
  if (d >= D) return;
  const typename Elem<DT>::T* kg = k + g * N * D + d;
  double s = 0.0;
  for (int64_t n = 0; n < N; ++n) s += (double)Elem<DT>::ld(kg, n * D);
  mean[g * D + d] = (float)(s / (double)N);
}

// ---- per-channel (column) quantisation over the key axis ----------------
// scale[g,d] = amax_n |x[g,n,d]| * fp32(1/127) (1 if 0); max is order-free.
// Blocks take (64 columns, a chunk of rows) and fold their max into the
// scale buffer with an integer atomic max on the (non-negative) float bits;
// a last pass turns the maxima into scales.
template <int DT>
__global__ void __launch_bounds__(MEAN_COLS * MEAN_PHASES)
col_amax_kernel(const typename Elem<DT>::T* __restrict__ x, unsigned int* __restrict__ amax_bits,
                int64_t N, int D) {
  __shared__ float part[MEAN_PHASES][MEAN_COLS];
  const int col = threadIdx.x % MEAN_COLS, ph = threadIdx.x / MEAN_COLS;
  const int64_t g = blockIdx.y;
  const int d = blockIdx.x * MEAN_COLS + col;
  const int64_t n0 = (int64_t)blockIdx.z * MEAN_CHUNK;
  const int64_t n1 = min(N, n0 + MEAN_CHUNK);
  float m = 0.f;
  if (d < D) {
    const typename Elem<DT>::T* xg = x + g * N * D + d;
#pragma unroll 4
    for (int64_t n = n0 + ph; n < n1; n += MEAN_PHASES) m = fmaxf(m, fabsf(Elem<DT>::ld(xg, n * D)));
  }
  part[ph][col] = m;
  __syncthreads();
  if (ph == 0 && d < D) {
#pragma unroll
    for (int p = 1; p < MEAN_PHASES; ++p) m = fmaxf(m, part[p][col]);
    atomicMax(amax_bits + g * D + d, __float_as_uint(m));
  }
}

__global__ void __launch_bounds__(256) col_scale_kernel(float* __restrict__ scale, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float s = scale[i] * (1.0f / 127.0f);  // scale holds the column max here
  scale[i] = (s == 0.f) ? 1.f : s;
}

__global__ void __launch_bounds__(256) u32_zero_kernel(unsigned int* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

template <int DT>
__global__ void __launch_bounds__(256)
col_quant_kernel(const typename Elem<DT>::T* __restrict__ x, const float* __restrict__ scale,
                 int8_t* __restrict__ q, int64_t N, int D, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int d = (int)(i % D);
  const int64_t g = i / ((int64_t)N * D);
  q[i] = code_of(Elem<DT>::ld(x, i), scale[g * D + d]);
}

}  // namespace
}  // namespace sl8

using namespace sl8;

extern "C" int sl8_quantize_i8_cols(const void* x, int dtype, int64_t G, int64_t N, int64_t D,
                                    int8_t* q, float* scale, void* stream) {
  clear_error();
  SL8_CHECK_ARG(dtype == SL8_DTYPE_F16 || dtype == SL8_DTYPE_BF16 || dtype == SL8_DTYPE_F32,
                "quantize_v_perchannel: input must be float16/bfloat16/float32");
  SL8_CHECK_ARG(G >= 0 && N >= 0 && D >= 0 && D < (1LL << 31), "quantize_v_perchannel: bad shape");
  if (G == 0 || D == 0) return SL8_OK;
  SL8_CHECK_ARG(x && q && scale, "quantize_v_perchannel: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nsc = G * D;
  const dim3 grid((unsigned)((D + MEAN_COLS - 1) / MEAN_COLS), (unsigned)G,
                  (unsigned)((N + MEAN_CHUNK - 1) / MEAN_CHUNK));
  const int64_t total = G * N * D;
  const unsigned qgrid = (unsigned)((total + 255) / 256);
  const unsigned sgrid = (unsigned)((nsc + 255) / 256);
  unsigned int* bits = reinterpret_cast<unsigned int*>(scale);
  u32_zero_kernel<<<sgrid, 256, 0, st>>>(bits, nsc);
  switch (dtype) {
    case SL8_DTYPE_F16:
      if (N) col_amax_kernel<SL8_DTYPE_F16><<<grid, MEAN_COLS * MEAN_PHASES, 0, st>>>(
          static_cast<const uint16_t*>(x), bits, N, (int)D);
      col_scale_kernel<<<sgrid, 256, 0, st>>>(scale, nsc);
      if (total) col_quant_kernel<SL8_DTYPE_F16><<<qgrid, 256, 0, st>>>(
          static_cast<const uint16_t*>(x), scale, q, N, (int)D, total);
      break;
    case SL8_DTYPE_BF16:
      if (N) col_amax_kernel<SL8_DTYPE_BF16><<<grid, MEAN_COLS * MEAN_PHASES, 0, st>>>(
          static_cast<const uint16_t*>(x), bits, N, (int)D);
      col_scale_kernel<<<sgrid, 256, 0, st>>>(scale, nsc);
      if (total) col_quant_kernel<SL8_DTYPE_BF16><<<qgrid, 256, 0, st>>>(
          static_cast<const uint16_t*>(x), scale, q, N, (int)D, total);
      break;
    default:
      if (N) col_amax_kernel<SL8_DTYPE_F32><<<grid, MEAN_COLS * MEAN_PHASES, 0, st>>>(
          static_cast<const float*>(x), bits, N, (int)D);
      col_scale_kernel<<<sgrid, 256, 0, st>>>(scale, nsc);
      if (total) col_quant_kernel<SL8_DTYPE_F32><<<qgrid, 256, 0, st>>>(
          static_cast<const float*>(x), scale, q, N, (int)D, total);
      break;
  }
  SL8_CHECK_LAUNCH("quantize_v_perchannel");
  return SL8_OK;
}

extern "C" const char* sl8_last_error(void) { return g_last_error.c_str(); }
extern "C" const char* sl8_version(void) { return "superl8-hip 0.1 gfx950"; }

extern "C" int sl8_quantize_i8_rowwise(const void* x, int x_dtype, int64_t M, int64_t K,
                                       int8_t* q, float* scale, void* stream) {
  clear_error();
  SL8_CHECK_ARG(x_dtype == SL8_DTYPE_F16 || x_dtype == SL8_DTYPE_BF16 || x_dtype == SL8_DTYPE_F32,
                "quantize_i8_rowwise input must be float16/bfloat16/float32");
  SL8_CHECK_ARG(M >= 0 && K >= 0 && K < (1LL << 31), "quantize_i8_rowwise: bad shape [%lld,%lld]",
                (long long)M, (long long)K);
  if (M == 0 || K == 0) return SL8_OK;
  SL8_CHECK_ARG(x && q && scale, "quantize_i8_rowwise: null pointer");
  SL8_CHECK_ARG((K & 3) != 0 || aligned(q, 4), "quantize_i8_rowwise: q must be 4-byte aligned");
  return dispatch_quant(x, x_dtype, nullptr, q, scale, M, 1, K, 1.0f,
                        static_cast<hipStream_t>(stream));
}

namespace sl8 {
namespace {

// ---------------------------------------------------------------------------
// Row-group quantisation (one scale per R consecutive rows of a [G][N][K]
// tensor, groups restarting at every G slice): the per-wavefront Q / per-tile
// K scheme of BASELINE config 5. One workgroup per group: pass 1 takes the
// amax of the (optionally mean-shifted, dtype-rounded) values over the R x K
// block, pass 2 writes the codes (the block is re-read from L2). The scale,
// safe value and code follow the row-wise contract above with the group's
// amax in place of the row's; every row of the group stores the group scale.
// ---------------------------------------------------------------------------
template <int DT, bool MEAN>
__global__ void __launch_bounds__(QTHREADS)
quant_row_groups_kernel(const typename Elem<DT>::T* __restrict__ x, const float* __restrict__ mean,
                        int8_t* __restrict__ q, float* __restrict__ scale, int64_t N, int K, int R,
                        float scale_mul) {
  using T = typename Elem<DT>::T;
  __shared__ float red[QTHREADS / 64];
  const int64_t g = blockIdx.y;                  // slice
  const int64_t r0 = (int64_t)blockIdx.x * R;    // first row of the group in the slice
  const int nr = (int)min((int64_t)R, N - r0);
  const T* xb = x + (g * N + r0) * K;
  const float* mr = MEAN ? mean + g * K : nullptr;
  const int total = nr * K;
  float amax = 0.f;
  for (int i = threadIdx.x; i < total; i += QTHREADS)
    amax = fmaxf(amax, fabsf(row_val<DT, MEAN>(xb + (i / K) * K, mr, i % K)));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = amax * (1.0f / 127.0f);
  const float safe = (s == 0.f) ? 1.f : s;
  for (int i = threadIdx.x; i < nr; i += QTHREADS) scale[g * N + r0 + i] = safe * scale_mul;
  int8_t* qb = q + (g * N + r0) * K;
  for (int i = threadIdx.x; i < total; i += QTHREADS)
    qb[i] = code_of(row_val<DT, MEAN>(xb + (i / K) * K, mr, i % K), safe);
}

}  // namespace
}  // namespace sl8

extern "C" int sl8_quantize_i8_row_groups(const void* x, int x_dtype, int64_t G, int64_t N,
                                          int64_t D, int64_t rows_per_group, const float* mean,
                                          float scale_mul, int8_t* q, float* scale, void* stream) {
  clear_error();
  SL8_CHECK_ARG(x_dtype == SL8_DTYPE_F16 || x_dtype == SL8_DTYPE_BF16 || x_dtype == SL8_DTYPE_F32,
                "quantize: input must be float16/bfloat16/float32");
  SL8_CHECK_ARG(G >= 0 && N >= 0 && D >= 0 && D < (1 << 20) && rows_per_group >= 1 &&
                    rows_per_group * D < (1LL << 30) && G < 65536,
                "quantize_row_groups: bad shape");
  if (G == 0 || N == 0 || D == 0) return SL8_OK;
  SL8_CHECK_ARG(x && q && scale, "quantize: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((N + rows_per_group - 1) / rows_per_group), (unsigned)G);
#define SL8_RG(DT, MN)                                                                          \
  quant_row_groups_kernel<DT, MN><<<grid, QTHREADS, 0, st>>>(                                   \
      static_cast<const typename Elem<DT>::T*>(x), mean, q, scale, N, (int)D, (int)rows_per_group, \
      scale_mul)
  if (mean) {
    if (x_dtype == SL8_DTYPE_F16) SL8_RG(SL8_DTYPE_F16, true);
    else if (x_dtype == SL8_DTYPE_BF16) SL8_RG(SL8_DTYPE_BF16, true);
    else SL8_RG(SL8_DTYPE_F32, true);
  } else {
    if (x_dtype == SL8_DTYPE_F16) SL8_RG(SL8_DTYPE_F16, false);
    else if (x_dtype == SL8_DTYPE_BF16) SL8_RG(SL8_DTYPE_BF16, false);
    else SL8_RG(SL8_DTYPE_F32, false);
  }
#undef SL8_RG
  SL8_CHECK_LAUNCH("quantize_row_groups");
  return SL8_OK;
}

extern "C" int sl8_quantize_i8_rows_centered(const void* x, int x_dtype, int64_t G, int64_t N,
                                             int64_t D, const float* mean, float scale_mul,
                                             int8_t* q, float* scale, void* stream) {
  clear_error();
  SL8_CHECK_ARG(x_dtype == SL8_DTYPE_F16 || x_dtype == SL8_DTYPE_BF16 || x_dtype == SL8_DTYPE_F32,
                "quantize: input must be float16/bfloat16/float32");
  SL8_CHECK_ARG(G >= 0 && N >= 0 && D >= 0 && D < (1LL << 31), "quantize: bad shape");
  if (G == 0 || N == 0 || D == 0) return SL8_OK;
  SL8_CHECK_ARG(x && q && scale, "quantize: null pointer");
  SL8_CHECK_ARG((D & 3) != 0 || aligned(q, 4), "quantize: q must be 4-byte aligned");
  return dispatch_quant(x, x_dtype, mean, q, scale, G * N, N, D, scale_mul,
                        static_cast<hipStream_t>(stream));
}

extern "C" size_t sl8_k_mean_workspace(int64_t G, int64_t D) {
  if (G <= 0 || D <= 0) return 0;
  return (size_t)(G * D) * sizeof(long long);
}

extern "C" int sl8_k_mean(const void* k, int dtype, int64_t G, int64_t N, int64_t D,
                          float* mean, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  SL8_CHECK_ARG(dtype == SL8_DTYPE_F16 || dtype == SL8_DTYPE_BF16 || dtype == SL8_DTYPE_F32,
                "k_mean: input must be float16/bfloat16/float32");
  SL8_CHECK_ARG(G >= 0 && N >= 0 && D >= 0 && D < (1LL << 31), "k_mean: bad shape");
  SL8_CHECK_ARG(N < (1LL << 23), "k_mean: N must be < 2^23 keys, got %lld", (long long)N);
  if (G == 0 || D == 0) return SL8_OK;
  SL8_CHECK_ARG(N > 0, "k_mean: mean over zero keys");
  SL8_CHECK_ARG(k && mean, "k_mean: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SL8_DTYPE_F16) {
    const size_t need = sl8_k_mean_workspace(G, D);
    SL8_CHECK_ARG(workspace && workspace_bytes >= need && aligned(workspace, 8),
                  "k_mean: workspace needs %zu bytes", need);
    unsigned long long* acc = static_cast<unsigned long long*>(workspace);
    const int64_t n = G * D;
    const unsigned ng = (unsigned)((n + 255) / 256);
    i64_zero_kernel<<<ng, 256, 0, st>>>(acc, n);
    const dim3 grid((unsigned)((D + MEAN_COLS - 1) / MEAN_COLS), (unsigned)G,
                    (unsigned)((N + MEAN_CHUNK - 1) / MEAN_CHUNK));
    k_mean_f16_kernel<<<grid, MEAN_COLS * MEAN_PHASES, 0, st>>>(static_cast<const uint16_t*>(k),
                                                                 acc, N, (int)D);
    k_mean_finish_kernel<<<ng, 256, 0, st>>>(acc, mean, n, N);
  } else {
    const dim3 grid((unsigned)((D + MEAN_COLS - 1) / MEAN_COLS), (unsigned)G);
    if (dtype == SL8_DTYPE_BF16)
      k_mean_seq_kernel<SL8_DTYPE_BF16><<<grid, MEAN_COLS, 0, st>>>(static_cast<const uint16_t*>(k),
                                                                    mean, N, (int)D);
    else
      k_mean_seq_kernel<SL8_DTYPE_F32><<<grid, MEAN_COLS, 0, st>>>(static_cast<const float*>(k),
                                                                   mean, N, (int)D);
  }
  SL8_CHECK_LAUNCH("k_mean");
  return SL8_OK;
}

// ---------------------------------------------------------------------------
// Outlier gate (reference superl8/quant/core.py:113-145): any row of Q with
// max|q| / (median|q| + 1e-10) > ratio (fp32) routes the call to full
// precision. One wave per row of D <= 64 E elements (lanes past D hold no
// element: they never count as "below" and add 0 to the max). The median is torch's
// lower median, the ((D-1)/2)-th smallest |q|, found exactly by a radix
// select on the fp32 bit patterns (non-negative floats order like their bits):
// 31 rounds of "how many elements lie below this prefix" (ballot + popcount).
// A row holding a NaN reports NaN for both and never fires, as in torch.
// ---------------------------------------------------------------------------
namespace sl8 {
namespace {

template <int DT, int E>
__global__ void __launch_bounds__(256)
q_gate_kernel(const void* __restrict__ q, int64_t rows, int D, float ratio,
              int32_t* __restrict__ flag, float* __restrict__ stats) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  uint32_t bits[E];
  float mx = 0.f;
  bool nan = false;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int c = e * 64 + lane;
    const int64_t i = row * D + (c < D ? c : 0);
    float x;
    if constexpr (DT == SL8_DTYPE_F32) x = static_cast<const float*>(q)[i];
    else x = u16_to_f<DT>(static_cast<const uint16_t*>(q)[i]);
    x = c < D ? fabsf(x) : 0.f;
    nan |= x != x;
    bits[e] = c < D ? __float_as_uint(x) : 0xFFFFFFFFu;
    mx = fmaxf(mx, x);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  const int K = (D - 1) / 2;
  uint32_t ans = 0;
  for (int b = 30; b >= 0; --b) {
    const uint32_t t = ans | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) cnt += __popcll(__ballot(bits[e] < t));
    if (cnt <= K) ans = t;
  }
  float med = __uint_as_float(ans);
  if (__ballot(nan)) {  // torch's amax and median both propagate NaN: the row never fires
    mx = __uint_as_float(0x7fc00000u);
    med = mx;
  }
  if (lane == 0) {
    if (stats) {
      stats[2 * row] = mx;
      stats[2 * row + 1] = med;
    }
    if (__fdiv_rn(mx, med + 1e-10f) > ratio) atomicOr(flag, 1);
  }
}

}  // namespace
}  // namespace sl8

extern "C" int sl8_q_outlier_gate(const void* q, int dtype, int64_t rows, int64_t D, float ratio,
                                  int32_t* flag, float* stats, void* stream) {
  clear_error();
  SL8_CHECK_ARG(rows >= 0 && D >= 1 && D <= 256,
                "fni8 outlier gate: head dim must be 1..256, got %lld", (long long)D);
  SL8_CHECK_ARG(dtype == SL8_DTYPE_F16 || dtype == SL8_DTYPE_BF16 || dtype == SL8_DTYPE_F32,
                "fni8 outlier gate: q must be float16, bfloat16 or float32");
  if (rows == 0) return SL8_OK;
  SL8_CHECK_ARG(q && flag, "fni8 outlier gate: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((rows + 3) / 4));
#define SL8_GATE(DT, E) q_gate_kernel<DT, E><<<grid, 256, 0, st>>>(q, rows, (int)D, ratio, flag, stats)
#define SL8_GATE_D(DT) \
  if (D <= 64) SL8_GATE(DT, 1); else if (D <= 128) SL8_GATE(DT, 2); else SL8_GATE(DT, 4);
  if (dtype == SL8_DTYPE_F16) { SL8_GATE_D(SL8_DTYPE_F16) }
  else if (dtype == SL8_DTYPE_BF16) { SL8_GATE_D(SL8_DTYPE_BF16) }
  else { SL8_GATE_D(SL8_DTYPE_F32) }
#undef SL8_GATE_D
#undef SL8_GATE
  SL8_CHECK_LAUNCH("outlier gate");
  return SL8_OK;
}

// ---------------------------------------------------------------------------
// Fused attention prologue for fp16 Q/K (reference superl8/quant/core.py
// quantize_qk + smooth_k, and the outlier gate of superl8/ops.py:115-147):
// two launches instead of six, Q read once, K read twice, no zeroing pass.
//
// Launch A: K-mean partials. Block (g, c) sums key rows [128c, 128c + 128)
//   of group g exactly in int64 fixed point (value * 2^24, decoded from the
//   fp16 bits) with 16-byte loads, all of a thread's rows in flight at once,
//   and stores its D partial sums; the mean is exact, hence independent of
//   the summation order. Block 0 also clears the gate flag.
// Launch B, two roles chosen per block:
//   * K: issues its key rows' loads, forms the group's mean from the C
//     partials meanwhile (int64 -> fp64 -> / N -> fp32, as sl8_k_mean; the
//     first block of each group also stores it), subtracts it from each row
//     with the fp16 rounding of torch.sub and quantises the row;
//   * Q: per-row int8 quantisation (scale * q_scale_mul) and, with a gate
//     ratio, the outlier decision for every row. f(x) = fl(max / fl(x + 1e-10))
//     is non-increasing in x >= 0, so f(median) > ratio iff more than (D-1)/2
//     of the row's |x| have f(|x|) > ratio: the row is decided exactly with
//     no median search (the division is needed only for elements within
//     2^-18 of max / ratio). A row holding a NaN never fires (torch's amax and
//     median are NaN there). A block with a firing row ORs 1 into the flag
//     (atomicOr), so the flag is set iff some row fires.
// ---------------------------------------------------------------------------
namespace sl8 {
namespace {

constexpr int PRO_CHUNK = 128;      // key rows per mean partial
constexpr int PRO_KROWS = 64;       // key rows per quantise block (each K block also forms its group's mean: 32 measured 1 us slower at config 2, 128 0.3 us)
constexpr int PRO_QBLOCKS_MAX = 16384;
constexpr int PRO_QP = 1;           // Q rows per thread per pass (1: measured fastest; more rows per thread cost occupancy)

// fp16 bits -> value * 2^24 as an exact integer (finite inputs: |result| < 2^40)
__device__ __forceinline__ long long f16_fixed24(uint32_t h) {
  const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
  const long long v = e ? (long long)(1024u + m) << (e - 1) : (long long)m;
  return (h & 0x8000u) ? -v : v;
}

template <int LPR>
__device__ __forceinline__ float group_max(float v) { return lane_group_max<LPR>(v); }
template <int LPR>
__device__ __forceinline__ int group_sum(int v) { return lane_group_sum<LPR>(v); }

__device__ __forceinline__ void unpack_h8(const uint4& raw, float* f) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) { f[2 * i] = h2f(w[i] & 0xFFFFu); f[2 * i + 1] = h2f(w[i] >> 16); }
}

// Eight codes clamp(rint(fl(x / safe))) without a division per element.
// |x| <= amax, so |x / safe| <= 127 * (1 + 2^-23) and, with inv = v_rcp_f32(safe)
// (at most 1 ulp from 1 / safe; safe >= 2^-24 / 127 here, a normal number),
// r = fl(x * inv) is within 128 * (2^-23 + 2^-24) = 1.5 * 2^-16 of x / safe,
// and fl(x / safe) within 2^-17 of it: |r - fl(x / safe)| < 2^-14. n = r
// rounded to nearest-even by the 1.5 * 2^23 magic constant; unless
// |r - n| > 0.5 - 2^-14 (r near a half-integer) both r and fl(x / safe)
// round to n. Lanes holding such an element (about 1e-4 of them) take the
// IEEE division, under a wave-uniform branch so the common path never
// executes it.
__device__ __forceinline__ uint2 codes8(const float* f, float safe) {
  const float inv = __builtin_amdgcn_rcpf(safe);
  constexpr float MAGIC = 12582912.f;  // 1.5 * 2^23
  float n[8];
  bool amb = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float r = f[e] * inv;
    n[e] = (r + MAGIC) - MAGIC;
    amb |= !(fabsf(r - n[e]) <= 0.5f - 0x1p-14f);  // also catches inf / NaN
  }
  if (__builtin_expect(__ballot(amb) != 0, 0)) {
    if (amb) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        n[e] = rintf(__fdiv_rn(f[e], safe));
        if (n[e] != n[e]) n[e] = -127.f;  // NaN: the clamp of fmaxf / fminf gives -127
      }
    }
  }
  // n is an integer in [-128, 128] (or the division's result): clamp as int
  uint32_t w[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int c[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) c[e] = __builtin_amdgcn_fmed3f(n[4 * i + e], -127.f, 127.f);
    // bytes 0 of c0..c3 -> one dword (v_perm_b32: selectors 0-3 pick the
    // second operand's bytes, 4-7 the first's, 0x0c a zero byte)
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)c[1], (uint32_t)c[0], 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)c[3], (uint32_t)c[2], 0x04000c0cu);
    w[i] = lo | hi;
  }
  return make_uint2(w[0], w[1]);
}

// A: exact int64 fixed-point K-mean partials of PRO_CHUNK-row chunks (one
// block per (group, chunk)); block 0 also clears the gate flag, which the Q
// blocks of B set.
template <int D>
__global__ void __launch_bounds__(256, 8)
prologue_a_kernel(const uint16_t* __restrict__ k, int64_t N, int C,
                  long long* __restrict__ part, int32_t* __restrict__ flag) {
  constexpr int LPR = D / 8;       // lanes per row, 8 elements (16 bytes) each
  constexpr int RPP = 256 / LPR;   // rows per block pass
  const int lane = threadIdx.x % LPR, sub = threadIdx.x / LPR;
  if (flag && blockIdx.x == 0 && threadIdx.x == 0) *flag = 0;
  __shared__ long long red[RPP][D];
  const int64_t g = blockIdx.x / C;
  const int c = blockIdx.x % C;
  const int64_t n0 = (int64_t)c * PRO_CHUNK, n1 = min(N, n0 + PRO_CHUNK);
  const uint16_t* kg = k + g * N * D + lane * 8;
  long long acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0;
  // every row load of the chunk is issued before any is summed (one round trip)
  constexpr int NIT = PRO_CHUNK / RPP;
  uint4 raw[NIT];
#pragma unroll
  for (int i = 0; i < NIT; ++i) {
    const int64_t n = n0 + sub + (int64_t)i * RPP;
    raw[i] = n < n1 ? *reinterpret_cast<const uint4*>(kg + n * D) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const uint32_t w[4] = {raw[it].x, raw[it].y, raw[it].z, raw[it].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += f16_fixed24(w[i] & 0xFFFFu);
      acc[2 * i + 1] += f16_fixed24(w[i] >> 16);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[sub][lane * 8 + e] = acc[e];
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += 256) {
    long long t = 0;
#pragma unroll 8
    for (int p = 0; p < RPP; ++p) t += red[p][d];
    part[(g * C + c) * D + d] = t;
  }
}

// B: the smoothed K rows (blocks [0, nkb): PRO_KROWS rows of group
// blockIdx / kbg each) and the Q rows with the outlier gate (the rest). The Q
// work does not depend on the mean, but sharing this launch keeps it off the
// critical path A -> mean -> B of the K side.
template <int D, bool GATE>
__global__ void __launch_bounds__(256)
prologue_b_kernel(const uint16_t* __restrict__ k, int64_t N, const long long* __restrict__ part,
                  int C, float* __restrict__ k_mean,
                  int8_t* __restrict__ k_i8, float* __restrict__ k_scale, int kbg, int nkb,
                  const uint16_t* __restrict__ q, int64_t qrows, float qmul, float ratio,
                  int8_t* __restrict__ q_i8, float* __restrict__ q_scale,
                  int32_t* __restrict__ flag) {
  constexpr int LPR = D / 8, RPP = 256 / LPR;
  const int lane = threadIdx.x % LPR, sub = threadIdx.x / LPR;
  if ((int)blockIdx.x < nkb) {
    constexpr int NP = PRO_KROWS / RPP;
    const int64_t g = blockIdx.x / kbg;
    const int64_t n0 = (int64_t)(blockIdx.x % kbg) * PRO_KROWS;
    const uint16_t* kg = k + g * N * D;
    uint4 raw[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int64_t n = n0 + i * RPP + sub;
      raw[i] = n < N ? reinterpret_cast<const uint4*>(kg + n * D)[lane] : make_uint4(0, 0, 0, 0);
    }
    // the group's mean from A's partials while the rows are in flight:
    // column d summed by PS threads over every PS-th partial, then in LDS
    constexpr int PS = 256 / D;
    __shared__ long long mred[PS][D];
    __shared__ float mean_s[D];
    {
      const int d = threadIdx.x % D, ps = threadIdx.x / D;
      const long long* pg = part + g * C * D + d;
      long long t = 0;
#pragma unroll 8
      for (int c = ps; c < C; c += PS) t += pg[(int64_t)c * D];
      mred[ps][d] = t;
    }
    __syncthreads();
    if (threadIdx.x < D) {
      long long t = 0;
#pragma unroll
      for (int p = 0; p < PS; ++p) t += mred[p][threadIdx.x];
      const float m = (float)(((double)t * 0x1p-24) / (double)N);
      mean_s[threadIdx.x] = m;
      if (blockIdx.x % kbg == 0) k_mean[g * D + threadIdx.x] = m;
    }
    __syncthreads();
    float mv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) mv[e] = mean_s[lane * 8 + e];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int64_t n = n0 + i * RPP + sub;
      const bool live = n < N;
      float f[8];
      unpack_h8(raw[i], f);
      float mx = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        f[e] = Elem<SL8_DTYPE_F16>::round(f[e] - mv[e]);
        mx = fmaxf(mx, fabsf(f[e]));
      }
      mx = group_max<LPR>(mx);
      const float s = mx * (1.0f / 127.0f);
      const float safe = (s == 0.f) ? 1.f : s;
      if (live) {
        if (lane == 0) k_scale[g * N + n] = safe;
        reinterpret_cast<uint2*>(k_i8 + (g * N + n) * D)[lane] = codes8(f, safe);
      }
    }
    return;
  }
  const int qb = blockIdx.x - nkb, nqb = gridDim.x - nkb;
  int fired = 0;
  const float rinv = 1.f / ratio;
  for (int64_t base = (int64_t)qb * RPP * PRO_QP; base < qrows;
       base += (int64_t)nqb * RPP * PRO_QP) {
    uint4 raw[PRO_QP];  // all of this thread's rows are fetched before any is processed
#pragma unroll
    for (int p = 0; p < PRO_QP; ++p) {
      const int64_t r = base + p * RPP + sub;
      raw[p] = r < qrows ? reinterpret_cast<const uint4*>(q + r * D)[lane] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < PRO_QP; ++p) {
      const int64_t r = base + p * RPP + sub;
      const bool live = r < qrows;
      float f[8];
      unpack_h8(raw[p], f);
      float mx = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(f[e]));
      mx = group_max<LPR>(mx);
      const float s = mx * (1.0f / 127.0f);
      const float safe = (s == 0.f) ? 1.f : s;
      if (live) {
        if (lane == 0) q_scale[r] = safe * qmul;
        reinterpret_cast<uint2*>(q_i8 + r * D)[lane] = codes8(f, safe);
      }
      if constexpr (GATE) {
        // y = fl(|x| + 1e-10) against t = max / ratio: far from t the exact test
        // fl(max / y) > ratio is decided by y < t; within 2^-18 of t (relative)
        // the IEEE division decides.
        // (t below 2^-100: every element takes the division.)
        const float t = mx * rinv;
        const bool tiny = t < 0x1p-100f;
        const float tlo = tiny ? 0.f : t * (1.f - 0x1p-18f);
        const float thi = tiny ? INFINITY : t * (1.f + 0x1p-18f);
        int cnt = 0, nan = 0;
        bool amb = false;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float a = fabsf(f[e]);
          nan |= a != a;
          const float y = a + 1e-10f;
          cnt += y < tlo;
          amb |= y >= tlo && y <= thi;
        }
        if (__builtin_expect(__ballot(amb) != 0, 0)) {
          if (amb) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float y = fabsf(f[e]) + 1e-10f;
              if (y >= tlo && y <= thi) cnt += __fdiv_rn(mx, y) > ratio;
            }
          }
        }
        cnt = group_sum<LPR>(cnt + (nan << 16));  // NaN count in the high half
        if (live && (cnt >> 16) == 0 && (cnt & 0xFFFF) > (D - 1) / 2) fired = 1;
      }
    }
  }
  if constexpr (GATE) {
    fired = __syncthreads_or(fired);
    if (fired && threadIdx.x == 0) atomicOr(flag, 1);  // cleared by A, earlier on the stream
  }
}

int prologue_nqb(int64_t qrows, int64_t D) {
  const int64_t rpp = 256 / (D / 8) * PRO_QP;
  return (int)std::min<int64_t>(PRO_QBLOCKS_MAX, (qrows + rpp - 1) / rpp);
}

}  // namespace
}  // namespace sl8

extern "C" size_t sl8_quantize_qk_workspace(int64_t BHq_M, int64_t G, int64_t N, int64_t D) {
  if (G <= 0 || N <= 0 || D <= 0) return 0;
  const int64_t C = (N + PRO_CHUNK - 1) / PRO_CHUNK;
  (void)BHq_M;  // the Q rows need no workspace (the gate sets the flag directly)
  return (size_t)(G * C * D) * sizeof(long long);  // the K-mean partials
}

extern "C" int sl8_quantize_qk(const void* q, const void* k, int dtype, int64_t qrows, int64_t G,
                               int64_t N, int64_t D, float q_scale_mul, float gate_ratio,
                               int8_t* q_i8, float* q_scale, int8_t* k_i8, float* k_scale,
                               float* k_mean, int32_t* gate_flag, void* workspace,
                               size_t workspace_bytes, void* stream) {
  clear_error();
  SL8_CHECK_ARG(dtype == SL8_DTYPE_F16, "fused prologue: q and k must be float16");
  SL8_CHECK_ARG(D == 64 || D == 128 || D == 256,
                "fused prologue: head dim must be 64/128/256, got %lld", (long long)D);
  SL8_CHECK_ARG(qrows > 0 && G > 0 && N > 0 && N < (1LL << 23),
                "fused prologue: bad shape (rows %lld, groups %lld, keys %lld)", (long long)qrows,
                (long long)G, (long long)N);
  SL8_CHECK_ARG(q && k && q_i8 && q_scale && k_i8 && k_scale && k_mean, "fused prologue: null pointer");
  SL8_CHECK_ARG(aligned(q, 16) && aligned(k, 16) && aligned(q_i8, 8) && aligned(k_i8, 8),
                "fused prologue: q/k must be 16-byte and codes 8-byte aligned");
  const bool gate = gate_ratio > 0.f;
  SL8_CHECK_ARG(!gate || gate_flag, "fused prologue: gate_flag required with a gate ratio");
  const size_t need = sl8_quantize_qk_workspace(qrows, G, N, D);
  SL8_CHECK_ARG(workspace && workspace_bytes >= need && aligned(workspace, 8),
                "fused prologue: workspace needs %zu bytes", need);
  const int C = (int)((N + PRO_CHUNK - 1) / PRO_CHUNK);
  const int64_t kbg = (N + PRO_KROWS - 1) / PRO_KROWS;  // quantise blocks per group
  SL8_CHECK_ARG(G * C < (1LL << 30) && G * kbg < (1LL << 30) && G < 65536,
                "fused prologue: too many key groups");
  const int nka = (int)(G * C), nkb = (int)(G * kbg), nqb = prologue_nqb(qrows, D);
  long long* part = static_cast<long long*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* qh = static_cast<const uint16_t*>(q);
  const uint16_t* kh = static_cast<const uint16_t*>(k);
  int32_t* fl = gate ? gate_flag : nullptr;
  // A (K-mean partials) -> B (the mean, K and Q rows, gate): the Q rows, the
  // bulk of the bytes, run beside the K rows in B instead of ahead of the mean
#define SL8_PRO(DD)                                                                              \
  do {                                                                                          \
    prologue_a_kernel<DD><<<nka, 256, 0, st>>>(kh, N, C, part, fl);                              \
    if (gate)                                                                                   \
      prologue_b_kernel<DD, true><<<nkb + nqb, 256, 0, st>>>(kh, N, part, C, k_mean, k_i8,      \
          k_scale, (int)kbg, nkb, qh, qrows, q_scale_mul, gate_ratio, q_i8, q_scale, fl);       \
    else                                                                                        \
      prologue_b_kernel<DD, false><<<nkb + nqb, 256, 0, st>>>(kh, N, part, C, k_mean, k_i8,     \
          k_scale, (int)kbg, nkb, qh, qrows, q_scale_mul, gate_ratio, q_i8, q_scale, fl);       \
  } while (0)
  if (D == 64) SL8_PRO(64);
  else if (D == 128) SL8_PRO(128);
  else SL8_PRO(256);
#undef SL8_PRO
  SL8_CHECK_LAUNCH("fused prologue");
  return SL8_OK;
}
