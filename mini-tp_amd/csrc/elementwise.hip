// Synthetic initialisation, embedding gather, RMSNorm, residual add, SwiGLU.
#include "common.h"
#include "kernels.h"

namespace minitp {

// ---------------------------------------------------------------------------
// Seeded generator (same spec as the CPU statement: integer splitmix64
// hashing, Marsaglia polar method, a log built from + - * / only). The
// double ops below use the _rn intrinsics so nothing is contracted.
#define GAMMA 0x9E3779B97F4A7C15ULL

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z ^= z >> 30;
  z *= 0xBF58476D1CE4E5B9ULL;
  z ^= z >> 27;
  z *= 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

uint64_t synth_key(uint64_t seed, uint64_t stream_id) {
  uint64_t z = seed * GAMMA + stream_id * 0xD1B54A32D192ED03ULL + 1ULL;
  z ^= z >> 30;
  z *= 0xBF58476D1CE4E5B9ULL;
  z ^= z >> 27;
  z *= 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

__device__ double det_log(double s) {
  uint64_t bits = (uint64_t)__double_as_longlong(s);
  int64_t e = (int64_t)((bits >> 52) & 0x7FFULL) - 1023;
  double m = __longlong_as_double((long long)((bits & 0x000FFFFFFFFFFFFFULL) | 0x3FF0000000000000ULL));
  if (m > 1.4142135623730951) {
    m = __dmul_rn(m, 0.5);
    e = e + 1;
  }
  double f = __ddiv_rn(__dsub_rn(m, 1.0), __dadd_rn(m, 1.0));
  double f2 = __dmul_rn(f, f);
  double p = __ddiv_rn(1.0, 23.0);
#pragma unroll
  for (int k = 10; k >= 0; --k) p = __dadd_rn(__dmul_rn(p, f2), __ddiv_rn(1.0, (double)(2 * k + 1)));
  return __dadd_rn(__dmul_rn((double)e, 0.6931471805599453), __dmul_rn(__dmul_rn(2.0, f), p));
}

__device__ double synth_normal(uint64_t key, uint64_t i) {
  for (uint64_t j = 0; j < 64; ++j) {
    uint64_t c = i * 64ULL + j;
    uint64_t h1 = mix64(key + (2ULL * c) * GAMMA);
    uint64_t h2 = mix64(key + (2ULL * c + 1ULL) * GAMMA);
    double x = __dsub_rn(__dmul_rn(__dmul_rn((double)(h1 >> 11), 0x1p-53), 2.0), 1.0);
    double y = __dsub_rn(__dmul_rn(__dmul_rn((double)(h2 >> 11), 0x1p-53), 2.0), 1.0);
    double s = __dadd_rn(__dmul_rn(x, x), __dmul_rn(y, y));
    if (s > 0.0 && s < 1.0) return __dmul_rn(x, __dsqrt_rn(__ddiv_rn(__dmul_rn(-2.0, det_log(s)), s)));
  }
  return 0.0;
}

template <typename T>
__global__ void fill_normal_kernel(T* dst, int64_t count, uint64_t key, double std_dev) {
  int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < count; i += stride) {
    float v = (float)__dmul_rn(std_dev, synth_normal(key, (uint64_t)i));
    store_f32<T>(dst, i, v);
  }
}

__global__ void fill_ids_kernel(int64_t* dst, int64_t count, uint64_t key, uint64_t vocab) {
  int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < count) dst[i] = (int64_t)(((mix64(key + (uint64_t)i * GAMMA) >> 32) * vocab) >> 32);
}

template <typename T>
__global__ void fill_kernel(T* dst, int64_t count, float value) {
  int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < count; i += stride) store_f32<T>(dst, i, value);
}

int launch_fill_normal(hipStream_t st, int dtype, void* dst, int64_t count, uint64_t seed, uint64_t sid,
                       double std_dev) {
  uint64_t key = synth_key(seed, sid);
  int grid = (int)std::min<int64_t>(cdiv(count, 256), 65536);
  if (dtype == MINITP_F32)
    fill_normal_kernel<float><<<grid, 256, 0, st>>>((float*)dst, count, key, std_dev);
  else
    fill_normal_kernel<bf16><<<grid, 256, 0, st>>>((bf16*)dst, count, key, std_dev);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

int launch_fill_ids(hipStream_t st, int64_t* dst, int64_t count, uint64_t seed, uint64_t sid, int64_t vocab) {
  uint64_t key = synth_key(seed, sid);
  fill_ids_kernel<<<(unsigned)cdiv(count, 256), 256, 0, st>>>(dst, count, key, (uint64_t)vocab);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

int launch_fill(hipStream_t st, int dtype, void* dst, int64_t count, float value) {
  int grid = (int)std::min<int64_t>(cdiv(count, 256), 65536);
  if (dtype == MINITP_F32)
    fill_kernel<float><<<grid, 256, 0, st>>>((float*)dst, count, value);
  else
    fill_kernel<bf16><<<grid, 256, 0, st>>>((bf16*)dst, count, value);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

// ---------------------------------------------------------------------------
// Embedding gather: one block per token, 16-byte copies.
template <typename T>
__global__ void embedding_kernel(const T* __restrict__ table, const int64_t* __restrict__ ids, int64_t ids_ld,
                                 int64_t T_, T* __restrict__ out, int64_t hidden, int64_t vocab) {
  int64_t n = blockIdx.x;  // token index in [0, B*T)
  int64_t b = n / T_, t = n % T_;
  int64_t id = ids[b * ids_ld + t];
  T* dst = out + n * hidden;
  if (id < 0 || id >= vocab) {
    for (int64_t i = threadIdx.x; i < hidden; i += blockDim.x) store_f32<T>(dst, i, __builtin_nanf(""));
    return;
  }
  const uint4* src = reinterpret_cast<const uint4*>(table + id * hidden);
  uint4* d4 = reinterpret_cast<uint4*>(dst);
  int64_t nv = hidden * (int64_t)sizeof(T) / 16;
  for (int64_t i = threadIdx.x; i < nv; i += blockDim.x) d4[i] = src[i];
}

int launch_embedding(hipStream_t st, int dtype, const void* table, const int64_t* ids, int64_t ids_ld, int64_t B,
                     int64_t T_, void* out, int64_t hidden, int64_t vocab) {
  if (B * T_ == 0) return MINITP_OK;
  if (dtype == MINITP_F32)
    embedding_kernel<float><<<(unsigned)(B * T_), 128, 0, st>>>((const float*)table, ids, ids_ld, T_, (float*)out,
                                                                  hidden, vocab);
  else
    embedding_kernel<bf16><<<(unsigned)(B * T_), 128, 0, st>>>((const bf16*)table, ids, ids_ld, T_, (bf16*)out,
                                                                 hidden, vocab);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

// ---------------------------------------------------------------------------
// RMSNorm, one block (256 threads) per row. Reference math (layer.py:39-42):
// xf = float(x); r = 1 / sqrt(sum(xf*xf) / H + eps); out = dtype((xf*r) * w).
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                      T* __restrict__ out, int64_t hidden, float eps) {
  __shared__ float red[4];
  const T* xr = x + blockIdx.x * hidden;
  T* orow = out + blockIdx.x * hidden;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < hidden; i += 256) {
    float v = load_f32<T>(xr, i);
    ss += mul_rn(v, v);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = (red[0] + red[1]) + (red[2] + red[3]);
  float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(tot, (float)hidden), eps)));
  for (int64_t i = threadIdx.x; i < hidden; i += 256) {
    float v = load_f32<T>(xr, i);
    store_f32<T>(orow, i, mul_rn(mul_rn(v, r), load_f32<T>(w, i)));
  }
}

int launch_rmsnorm(hipStream_t st, int dtype, const void* x, const void* w, void* out, int64_t rows, int64_t hidden,
                   float eps) {
  if (rows == 0) return MINITP_OK;
  if (dtype == MINITP_F32)
    rmsnorm_kernel<float><<<(unsigned)rows, 256, 0, st>>>((const float*)x, (const float*)w, (float*)out, hidden, eps);
  else
    rmsnorm_kernel<bf16><<<(unsigned)rows, 256, 0, st>>>((const bf16*)x, (const bf16*)w, (bf16*)out, hidden, eps);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

// Residual add then RMSNorm of the sum, one block per row (layer.py:61-64
// then 39-42): x = dtype(x + delta) in place, out = RMSNorm(x). Each thread
// reads and writes only its own elements, so out may alias delta.
template <typename T>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(T* x, const T* delta, const T* __restrict__ w, T* out,
                                                          int64_t hidden, float eps) {
  __shared__ float red[4];
  T* xr = x + blockIdx.x * hidden;
  const T* dr = delta + blockIdx.x * hidden;
  T* orow = out + blockIdx.x * hidden;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < hidden; i += 256) {
    const float v = round_to<T>(add_rn(load_f32<T>(xr, i), load_f32<T>(dr, i)));
    store_f32<T>(xr, i, v);
    ss += mul_rn(v, v);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = (red[0] + red[1]) + (red[2] + red[3]);
  float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(tot, (float)hidden), eps)));
  for (int64_t i = threadIdx.x; i < hidden; i += 256) {
    float v = load_f32<T>(xr, i);
    store_f32<T>(orow, i, mul_rn(mul_rn(v, r), load_f32<T>(w, i)));
  }
}

// bf16 rows of hidden % 8 == 0: the same math in 16-byte pieces (8 elements per
// load and store; a thread's elements are whole pieces).
// PART: delta is the split-K partial product itself (the sum over the splits
// rounded to bf16 as gemm_reduce_kernel stores it), not a bf16 row.
template <bool PART>
__global__ __launch_bounds__(256) void add_rmsnorm8_kernel(bf16* x, const bf16* delta, Partials dp,
                                                           const bf16* __restrict__ w, bf16* out, int64_t hidden,
                                                           float eps) {
  __shared__ float red[4];
  uint4* xr = reinterpret_cast<uint4*>(x + blockIdx.x * hidden);
  const uint4* dr = reinterpret_cast<const uint4*>(delta + blockIdx.x * hidden);
  uint4* orow = reinterpret_cast<uint4*>(out + blockIdx.x * hidden);
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  const int64_t n8 = hidden / 8;
  float ss = 0.f;
  for (int64_t c = threadIdx.x; c < n8; c += 256) {
    float a[8], d[8];
    unpack16(xr[c], a, (bf16*)nullptr);
    if constexpr (PART) {
      float v[8];
      sum_partials8(dp, blockIdx.x, c * 8, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) d[e] = round_to<bf16>(v[e] + 0.f);
    } else {
      unpack16(dr[c], d, (bf16*)nullptr);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = round_to<bf16>(add_rn(a[e], d[e]));
      ss += mul_rn(a[e], a[e]);
    }
    xr[c] = make_uint4(pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(a[4], a[5]),
                       pack_bf16x2(a[6], a[7]));
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = (red[0] + red[1]) + (red[2] + red[3]);
  float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(tot, (float)hidden), eps)));
  for (int64_t c = threadIdx.x; c < n8; c += 256) {
    float a[8], wf[8], o[8];
    unpack16(xr[c], a, (bf16*)nullptr);
    unpack16(wr[c], wf, (bf16*)nullptr);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = mul_rn(mul_rn(a[e], r), wf[e]);
    orow[c] = make_uint4(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]), pack_bf16x2(o[4], o[5]),
                         pack_bf16x2(o[6], o[7]));
  }
}

int launch_add_rmsnorm(hipStream_t st, int dtype, void* x, const void* delta, const void* w, void* out, int64_t rows,
                       int64_t hidden, float eps) {
  if (rows == 0) return MINITP_OK;
  if (dtype == MINITP_BF16 && hidden % 8 == 0 && aligned16(x) && aligned16(delta) && aligned16(w) && aligned16(out)) {
    add_rmsnorm8_kernel<false><<<(unsigned)rows, 256, 0, st>>>((bf16*)x, (const bf16*)delta, Partials{}, (const bf16*)w,
                                                               (bf16*)out, hidden, eps);
    MINITP_LAUNCH_CHECK();
    return MINITP_OK;
  }
  if (dtype == MINITP_F32)
    add_rmsnorm_kernel<float><<<(unsigned)rows, 256, 0, st>>>((float*)x, (const float*)delta, (const float*)w,
                                                              (float*)out, hidden, eps);
  else
    add_rmsnorm_kernel<bf16><<<(unsigned)rows, 256, 0, st>>>((bf16*)x, (const bf16*)delta, (const bf16*)w, (bf16*)out,
                                                             hidden, eps);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

// ---------------------------------------------------------------------------
template <typename T>
__global__ void add_kernel(const T* a, const T* b, T* out, int64_t n, int64_t period) {
  int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) store_f32<T>(out, i, add_rn(load_f32<T>(a, i), load_f32<T>(b, i % period)));
}

int launch_add(hipStream_t st, int dtype, const void* a, const void* b, void* out, int64_t n, int64_t b_period) {
  if (n == 0) return MINITP_OK;
  int grid = (int)std::min<int64_t>(cdiv(n, 256), 65536);
  if (dtype == MINITP_F32)
    add_kernel<float><<<grid, 256, 0, st>>>((const float*)a, (const float*)b, (float*)out, n, b_period);
  else
    add_kernel<bf16><<<grid, 256, 0, st>>>((const bf16*)a, (const bf16*)b, (bf16*)out, n, b_period);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

template <typename T>
__global__ void silu_mul_kernel(const T* gate, const T* up, int64_t ld_in, T* out, int64_t ld_out, int64_t rows,
                                int64_t n) {
  int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  int64_t total = rows * n;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < total; i += stride) {
    int64_t r = i / n, c = i % n;
    float g = load_f32<T>(gate, r * ld_in + c);
    float u = load_f32<T>(up, r * ld_in + c);
    store_f32<T>(out, r * ld_out + c, swiglu<T>(g, u));
  }
}

// bf16, 8 elements per thread through 16-byte loads and stores (rows of n % 8
// == 0 elements, 16-byte aligned row starts); same math as silu_mul_kernel.
// PART: gate and up are the split-K partial product of the [gate; up]
// weight ([S][rows][2 n]), each sum rounded to bf16 as the GEMM stores it.
template <bool PART>
__global__ void silu_mul8_kernel(const bf16* gate, const bf16* up, int64_t ld_in, Partials gp, bf16* out,
                                 int64_t ld_out, int64_t rows, int64_t n) {
  const int64_t n8 = n / 8, total = rows * n8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / n8, c = (i % n8) * 8;
    float g[8], u[8], o[8];
    if constexpr (PART) {
      float vg[8], vu[8];
      sum_partials8(gp, r, c, vg);
      sum_partials8(gp, r, n + c, vu);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        g[e] = round_to<bf16>(vg[e] + 0.f);
        u[e] = round_to<bf16>(vu[e] + 0.f);
      }
    } else {
      const uint4 gv = *reinterpret_cast<const uint4*>(gate + r * ld_in + c);
      const uint4 uv = *reinterpret_cast<const uint4*>(up + r * ld_in + c);
      unpack16(gv, g, (bf16*)nullptr);
      unpack16(uv, u, (bf16*)nullptr);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = swiglu<bf16>(g[e], u[e]);
    *reinterpret_cast<uint4*>(out + r * ld_out + c) =
        make_uint4(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]), pack_bf16x2(o[4], o[5]), pack_bf16x2(o[6], o[7]));
  }
}

int launch_silu_mul(hipStream_t st, int dtype, const void* gate, const void* up, int64_t ld_in, void* out,
                    int64_t ld_out, int64_t rows, int64_t n) {
  if (rows * n == 0) return MINITP_OK;
  const bool vec = dtype == MINITP_BF16 && n % 8 == 0 && ld_in % 8 == 0 && ld_out % 8 == 0 && aligned16(gate) &&
                   aligned16(up) && aligned16(out);
  if (vec) {
    const int grid8 = (int)std::min<int64_t>(cdiv(rows * (n / 8), 256), 65536);
    silu_mul8_kernel<false><<<grid8, 256, 0, st>>>((const bf16*)gate, (const bf16*)up, ld_in, Partials{}, (bf16*)out,
                                                   ld_out, rows, n);
    MINITP_LAUNCH_CHECK();
    return MINITP_OK;
  }
  int grid = (int)std::min<int64_t>(cdiv(rows * n, 256), 65536);
  if (dtype == MINITP_F32)
    silu_mul_kernel<float><<<grid, 256, 0, st>>>((const float*)gate, (const float*)up, ld_in, (float*)out, ld_out,
                                                 rows, n);
  else
    silu_mul_kernel<bf16><<<grid, 256, 0, st>>>((const bf16*)gate, (const bf16*)up, ld_in, (bf16*)out, ld_out, rows,
                                                n);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

int launch_add_rmsnorm_partials(hipStream_t st, void* x, const Partials& delta, const void* w, void* out,
                                int64_t hidden, float eps) {
  if (delta.M == 0) return MINITP_OK;
  if (delta.N != hidden || hidden % 8 != 0 || delta.S < 1 || !aligned16(x) || !aligned16(delta.p) || !aligned16(w) ||
      !aligned16(out)) {
    set_error("add_rmsnorm from partials: hidden %lld, partial width %lld", (long long)hidden, (long long)delta.N);
    return MINITP_ERR_UNSUPPORTED;
  }
  add_rmsnorm8_kernel<true><<<(unsigned)delta.M, 256, 0, st>>>((bf16*)x, nullptr, delta, (const bf16*)w, (bf16*)out,
                                                              hidden, eps);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

int launch_silu_mul_partials(hipStream_t st, const Partials& gu, void* out, int64_t ld_out, int64_t n) {
  if (gu.M * n == 0) return MINITP_OK;
  if (gu.N != 2 * n || n % 8 != 0 || ld_out % 8 != 0 || gu.S < 1 || !aligned16(gu.p) || !aligned16(out)) {
    set_error("silu_mul from partials: n %lld, partial width %lld", (long long)n, (long long)gu.N);
    return MINITP_ERR_UNSUPPORTED;
  }
  const int grid8 = (int)std::min<int64_t>(cdiv(gu.M * (n / 8), 256), 65536);
  silu_mul8_kernel<true><<<grid8, 256, 0, st>>>(nullptr, nullptr, 0, gu, (bf16*)out, ld_out, gu.M, n);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

__global__ void cast_f32_bf16_kernel(const float* in, uint16_t* out, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += stride) out[i] = f32_to_bf16(in[i]);
}

int launch_cast_f32_bf16(hipStream_t st, const float* in, void* out, int64_t n) {
  if (n == 0) return MINITP_OK;
  const int grid = (int)std::min<int64_t>(cdiv(n, 256), 65536);
  cast_f32_bf16_kernel<<<grid, 256, 0, st>>>(in, (uint16_t*)out, n);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

}  // namespace minitp
