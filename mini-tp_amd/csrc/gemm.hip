// Prefill / batched linear layers: y[M, N] = epilogue(x[M, K] W[N, K]^T (+ bias)).
//
// MFMA tiling for CDNA (wave64): a 256-thread block owns a 128 x 128 output
// tile; its 4 waves form a 2 x 2 grid of 64 x 64 wave tiles, each a 2 x 2 set
// of 32 x 32 MFMA accumulators (16 fp32 registers per lane each). K advances
// in 64-byte slabs (32 bf16 or 16 fp32) staged in LDS; both operands are
// K-contiguous in memory (x rows and W rows), which is the layout the MFMA
// A/B fragments want, so no transpose is needed anywhere.
//   bf16: v_mfma_f32_32x32x8bf16_1k (A/B: 4 bf16 per lane, k = 4*(lane/32)+i)
//   fp32: v_mfma_f32_32x32x2f32     (A/B: 1 float per lane, k = lane/32)
// Accumulator layout: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4,
// column l%32.
#include "common.h"
#include "kernels.h"

namespace minitp {

namespace {

constexpr int BM = 128, BN = 128;
constexpr int SLAB = 64;  // bytes of K per LDS stage per row
constexpr int PADB = 16;  // row padding (bytes) against LDS bank conflicts
constexpr int ROWB = SLAB + PADB;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma;

template <>
struct Mfma<bf16> {
  static constexpr int KSTEP = 8;  // k per instruction
  __device__ static f32x16 step(const char* a_row, const char* b_row, int ks, int lane, f32x16 c) {
    const int off = (ks * KSTEP + (lane >> 5) * 4) * 2;
    s16x4 a = *reinterpret_cast<const s16x4*>(a_row + off);
    s16x4 b = *reinterpret_cast<const s16x4*>(b_row + off);
    return __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<float> {
  static constexpr int KSTEP = 2;
  __device__ static f32x16 step(const char* a_row, const char* b_row, int ks, int lane, f32x16 c) {
    const int off = (ks * KSTEP + (lane >> 5)) * 4;
    float a = *reinterpret_cast<const float*>(a_row + off);
    float b = *reinterpret_cast<const float*>(b_row + off);
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

template <typename T, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const T* __restrict__ x, int64_t ldx, const T* __restrict__ w,
                                                   const T* __restrict__ bias, T* y, int64_t ldy, const T* aux,
                                                   int64_t M, int64_t N, int64_t K, const StepState* state) {
  if (state != nullptr) y = (T*)state->args.logits;
  __shared__ __attribute__((aligned(16))) char As[BM * ROWB];
  __shared__ __attribute__((aligned(16))) char Bs[BN * ROWB];
  constexpr int V = Vec<T>::N;              // elements per 16 B
  constexpr int SLAB_K = SLAB / sizeof(T);  // elements of K per stage
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  for (int64_t k0 = 0; k0 < K; k0 += SLAB_K) {
    // stage: 128 rows x 4 chunks of 16 B for each operand = 2 chunks / thread
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = tid + h * 256, row = c >> 2, kc = c & 3;
      const int64_t k = k0 + kc * V;
      uint4 va = make_uint4(0, 0, 0, 0), vb = make_uint4(0, 0, 0, 0);
      if (m0 + row < M && k < K) va = *reinterpret_cast<const uint4*>(x + (m0 + row) * ldx + k);
      if (n0 + row < N && k < K) vb = load_stream16(reinterpret_cast<const uint4*>(w + (n0 + row) * K + k));
      *reinterpret_cast<uint4*>(As + row * ROWB + kc * 16) = va;
      *reinterpret_cast<uint4*>(Bs + row * ROWB + kc * 16) = vb;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < SLAB_K / Mfma<T>::KSTEP; ++ks) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const char* a_row = As + (wm * 64 + i * 32 + (lane & 31)) * ROWB;
          const char* b_row = Bs + (wn * 64 + j * 32 + (lane & 31)) * ROWB;
          acc[i][j] = Mfma<T>::step(a_row, b_row, ks, lane, acc[i][j]);
        }
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn * 64 + j * 32 + (lane & 31);
      if (col >= N) continue;
      const float bcol = (EPI == MINITP_EPI_NONE && bias != nullptr) ? load_f32<T>(bias, col) : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row >= M) continue;
        const float v = acc[i][j][r];
        if constexpr (EPI == MINITP_EPI_RESID)
          store_f32<T>(y, row * ldy + col, add_rn(load_f32<T>(aux, row * ldy + col), round_to<T>(v)));
        else
          store_f32<T>(y, row * ldy + col, v + bcol);
      }
    }
}

template <typename T>
int gemm_typed(hipStream_t st, const void* x, int64_t ldx, const void* w, const void* bias, void* y, int64_t ldy,
               int64_t M, int64_t N, int64_t K, int epi, const void* aux, const StepState* state) {
  dim3 grid((unsigned)cdiv(N, BN), (unsigned)cdiv(M, BM));
  if (epi == MINITP_EPI_RESID)
    hipLaunchKernelGGL((gemm_kernel<T, MINITP_EPI_RESID>), grid, dim3(256), 0, st, (const T*)x, ldx, (const T*)w,
                       (const T*)bias, (T*)y, ldy, (const T*)aux, M, N, K, state);
  else
    hipLaunchKernelGGL((gemm_kernel<T, MINITP_EPI_NONE>), grid, dim3(256), 0, st, (const T*)x, ldx, (const T*)w,
                       (const T*)bias, (T*)y, ldy, (const T*)aux, M, N, K, state);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

}  // namespace

int launch_gemm(hipStream_t st, int dtype, const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                int64_t ldy, int64_t M, int64_t N, int64_t K, int epi, const void* aux, const StepState* state) {
  if (M == 0 || N == 0) return MINITP_OK;
  if (epi != MINITP_EPI_NONE && epi != MINITP_EPI_RESID) {
    set_error("gemm: epilogue %d not supported (split SwiGLU runs as its own kernel)", epi);
    return MINITP_ERR_UNSUPPORTED;
  }
  return dtype == MINITP_F32 ? gemm_typed<float>(st, x, ldx, w, bias, y, ldy, M, N, K, epi, aux, state)
                             : gemm_typed<bf16>(st, x, ldx, w, bias, y, ldy, M, N, K, epi, aux, state);
}

}  // namespace minitp
