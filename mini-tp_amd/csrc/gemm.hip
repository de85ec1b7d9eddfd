// Prefill / batched linear layers: y[M, N] = epilogue(x[M, K] W[N, K]^T (+ bias)).
//
// MFMA tiling for CDNA (wave64): a 256-thread block owns a BM x BN output
// tile (128 x 128 for large M, 64 x 64 when M is small); its 4 waves form a
// 2 x 2 grid of wave tiles made of 32 x 32 MFMA accumulators (16 fp32
// registers per lane each). Both operands are K-contiguous in memory (x rows
// and W rows), the layout the MFMA A/B fragments want, so nothing is
// transposed. K advances in chunks of 256 bytes per row staged in LDS; the
// global loads of the next DEPTH chunks are in flight (in registers) while a
// chunk's MFMAs run. The loads
// are buffer loads whose lanes past the matrix (rows beyond M or N, K beyond
// the split) get an out-of-range offset and read zeros: no load sits behind
// a branch, so the compiler can count them precisely instead of waiting for
// all of them before the next ones issue. Rows are padded by 16 bytes in LDS
// to spread the MFMA fragment reads over the banks.
//   bf16: v_mfma_f32_32x32x16_bf16 (A/B: 8 bf16 per lane, k = 8*(lane/32)+i)
//   fp32: v_mfma_f32_32x32x2f32     (A/B: 1 float per lane, k = lane/32)
// Accumulator layout: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4,
// column l%32.
//
// Small M (prefill of one short prompt, batched decode) leaves few output
// tiles, so K is split over blockIdx.z: each split writes fp32 partial sums
// to a workspace and gemm_reduce_kernel adds them in split order (a fixed
// order, so results do not depend on timing) and applies the epilogue.
#include "common.h"
#include "kernels.h"

namespace minitp {

namespace {

constexpr int OUT_PARTIAL = 100;  // epilogue: fp32 split-K partials
// epilogue: SwiGLU of a [gate; up] weight (2N rows): tile column bx holds
// outputs [bx BN / 2, + BN / 2), its first BN / 2 B rows the gate rows and
// the rest the matching up rows, so waves wn = 0 hold gate and wn = 1 up
constexpr int OUT_SWIGLU = 101;
constexpr uint32_t OOB = 0xffffffffu;  // lane offset that reads zeros

template <int AUX>
__device__ __forceinline__ uint4 gemm_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
  return make_uint4(v.x, v.y, v.z, v.w);
}
// weight loads of gemm_kernel: plain (non-temporal measured slower: 0.5B
// 128-token TTFT 1.41-1.42 against 1.38 ms, 7B 512 tokens 11.55 against 11.28)
#ifndef MINITP_GEMM_NT_LOADS
#define MINITP_GEMM_NT_LOADS 0
#endif
constexpr int GEMM_W_AUX = MINITP_GEMM_NT_LOADS ? 2 : 0;
// chunks in flight: register budget of the prefetch (LA + LB uint4 each)
// (one chunk ahead measured best at the 0.5B prompt and 7B prefill shapes;
// two to four chunks were slower, also in a form whose loop the compiler
// counts exactly, waiting only for the chunk it stashes next)
#ifndef MINITP_GEMM_DEPTH_LARGE
#define MINITP_GEMM_DEPTH_LARGE 1
#endif
#ifndef MINITP_GEMM_DEPTH_SMALL
#define MINITP_GEMM_DEPTH_SMALL 1
#endif
// output tile of the small-M GEMMs (M < 512)
#ifndef MINITP_GEMM_SMALL_BM
#define MINITP_GEMM_SMALL_BM 64
#endif
#ifndef MINITP_GEMM_SMALL_BN
#define MINITP_GEMM_SMALL_BN 64
#endif
template <int BM>
constexpr int depth() {
  return BM >= 128 ? MINITP_GEMM_DEPTH_LARGE : MINITP_GEMM_DEPTH_SMALL;
}
// bytes of K per row per LDS chunk: 256 for 64 x 64 tiles, 128 for 128 x 128
// (both operand tiles of a chunk stay under 40 KiB of LDS)
template <int BM>
constexpr int chunk_bytes() {
  return BM >= 128 ? 128 : 256;
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T>
struct Mfma;

typedef __bf16 bf16x8_k __attribute__((ext_vector_type(8)));
// gfx950's 32x32x16: lane l holds A[l % 32][8 (l / 32) .. + 7] and the same
// k range of B column l % 32, one 16-byte LDS read each
template <>
struct Mfma<bf16> {
  static constexpr int KSTEP = 16;  // k per instruction
  __device__ static f32x16 step(const char* a_row, const char* b_row, int ks, int lane, f32x16 c) {
    const int off = (ks * KSTEP + (lane >> 5) * 8) * 2;
    const bf16x8_k a = *reinterpret_cast<const bf16x8_k*>(a_row + off);
    const bf16x8_k b = *reinterpret_cast<const bf16x8_k*>(b_row + off);
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
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

// Block (bx, by, z): output tile (by * BM, bx * BN), K range [z kper, (z + 1)
// kper). kper is a multiple of the chunk (KCB bytes).
template <typename T, int BM, int BN, int OUT>
__global__ __launch_bounds__(256) void gemm_kernel(const T* __restrict__ x, int64_t ldx, const T* __restrict__ w,
                                                   const T* __restrict__ bias, T* y, int64_t ldy, const T* aux,
                                                   float* part, int64_t M, int64_t N, int64_t K, int64_t kper,
                                                   const StepState* state) {
  if (state != nullptr) y = (T*)state->args.logits;
  constexpr int KCB = chunk_bytes<BM>(), ROWB = KCB + 16;
  constexpr int V = Vec<T>::N;          // elements per 16 B
  constexpr int KCE = KCB / sizeof(T);  // elements of K per chunk
  constexpr int CPR = KCB / 16;         // 16-byte pieces per row per chunk
  constexpr int LA = BM * CPR / 256, LB = BN * CPR / 256;  // pieces per thread
  constexpr int FM = BM / 64, FN = BN / 64;                // 32 x 32 fragments per wave
  __shared__ __attribute__((aligned(16))) char As[BM * ROWB];
  __shared__ __attribute__((aligned(16))) char Bs[BN * ROWB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t kb = (int64_t)blockIdx.z * kper;
  const int64_t ke = kb + kper < K ? kb + kper : K;

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  constexpr int DEPTH = depth<BM>();
  constexpr int ES = (int)sizeof(T);
  // x rows [0, M) and W rows [0, N) as buffers; a lane's piece is read only
  // when its row exists and its K lies inside this block's split
  const __amdgpu_buffer_rsrc_t xr = span_rsrc(x, (uint32_t)(((M - 1) * ldx + K) * ES));
  const __amdgpu_buffer_rsrc_t wr = span_rsrc(w, (uint32_t)((OUT == OUT_SWIGLU ? 2 : 1) * N * K * ES));
  uint4 ra[DEPTH][LA], rb[DEPTH][LB];
  auto load = [&](int64_t k0, uint4(&a)[LA], uint4(&bb)[LB]) {
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int c = tid + i * 256, row = c / CPR, pc = c % CPR;
      const int64_t k = k0 + pc * V;
      const bool ok = m0 + row < M && k < ke;
      a[i] = gemm_load16<0>(xr, ok ? (uint32_t)(((m0 + row) * ldx + k) * ES) : OOB);
    }
#pragma unroll
    for (int i = 0; i < LB; ++i) {
      const int c = tid + i * 256, row = c / CPR, pc = c % CPR;
      const int64_t k = k0 + pc * V;
      int64_t wrow = n0 + row;
      bool ok = wrow < N && k < ke;
      if constexpr (OUT == OUT_SWIGLU) {
        const int64_t j = (int64_t)blockIdx.x * (BN / 2) + row % (BN / 2);
        wrow = row < BN / 2 ? j : N + j;
        ok = j < N && k < ke;
      }
      bb[i] = gemm_load16<GEMM_W_AUX>(wr, ok ? (uint32_t)((wrow * K + k) * ES) : OOB);
    }
  };
  auto stash = [&](const uint4(&a)[LA], const uint4(&bb)[LB]) {
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int c = tid + i * 256, row = c / CPR, pc = c % CPR;
      *reinterpret_cast<uint4*>(As + row * ROWB + pc * 16) = a[i];
    }
#pragma unroll
    for (int i = 0; i < LB; ++i) {
      const int c = tid + i * 256, row = c / CPR, pc = c % CPR;
      *reinterpret_cast<uint4*>(Bs + row * ROWB + pc * 16) = bb[i];
    }
  };

  // chunk c of the split lives in register slot c % DEPTH (loads past the
  // split read zeros and are never stashed)
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) load(kb + (int64_t)d * KCE, ra[d], rb[d]);
  for (int64_t k0 = kb; k0 < ke; k0 += (int64_t)DEPTH * KCE) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int64_t kc = k0 + (int64_t)d * KCE;
      if (kc >= ke) break;
      stash(ra[d], rb[d]);
      __syncthreads();
      if (kc + DEPTH * KCE < ke) load(kc + (int64_t)DEPTH * KCE, ra[d], rb[d]);  // in flight for later chunks
#pragma unroll
      for (int ks = 0; ks < KCE / Mfma<T>::KSTEP; ++ks) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            const char* a_row = As + (wm * (BM / 2) + i * 32 + (lane & 31)) * ROWB;
            const char* b_row = Bs + (wn * (BN / 2) + j * 32 + (lane & 31)) * ROWB;
            acc[i][j] = Mfma<T>::step(a_row, b_row, ks, lane, acc[i][j]);
          }
      }
      __syncthreads();
    }
  }

  if constexpr (OUT == OUT_SWIGLU) {
    // the up waves hand their accumulators to the gate waves through LDS
    // (free after the last chunk's barrier): [wm][i][j][r][lane]
    float* xch = reinterpret_cast<float*>(As);
    static_assert(2 * FM * FN * 16 * 64 * 4 <= BM * ROWB, "exchange fits the A tile");
    if (wn == 1) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) xch[(((wm * FM + i) * FN + j) * 16 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (wn == 1) return;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int64_t col = (int64_t)blockIdx.x * (BN / 2) + j * 32 + (lane & 31);
        if (col >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (row >= M) continue;
          const float g = round_to<T>(acc[i][j][r] + 0.f);
          const float u = round_to<T>(xch[(((wm * FM + i) * FN + j) * 16 + r) * 64 + lane] + 0.f);
          store_f32<T>(y, row * ldy + col, swiglu<T>(g, u));
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t col = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
      if (col >= N) continue;
      const float bcol = (OUT == MINITP_EPI_NONE && bias != nullptr) ? load_f32<T>(bias, col) : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row >= M) continue;
        const float v = acc[i][j][r];
        if constexpr (OUT == OUT_PARTIAL)
          part[((int64_t)blockIdx.z * M + row) * N + col] = v;
        else if constexpr (OUT == MINITP_EPI_RESID)
          store_f32<T>(y, row * ldy + col, add_rn(load_f32<T>(aux, row * ldy + col), round_to<T>(v)));
        else
          store_f32<T>(y, row * ldy + col, v + bcol);
      }
    }
}

// y = epilogue(sum over the S splits of part[s][M][N]), splits added in order.
template <typename T, int EPI>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float* __restrict__ part, int S, const T* bias, T* y,
                                                          int64_t ldy, const T* aux, int64_t M, int64_t N,
                                                          const StepState* state) {
  if (state != nullptr) y = (T*)state->args.logits;
  const int64_t MN = M * N;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < MN; e += (int64_t)gridDim.x * blockDim.x) {
    float v = part[e];
    for (int s = 1; s < S; ++s) v += part[s * MN + e];
    const int64_t row = e / N, col = e % N;
    if constexpr (EPI == MINITP_EPI_RESID)
      store_f32<T>(y, row * ldy + col, add_rn(load_f32<T>(aux, row * ldy + col), round_to<T>(v)));
    else
      store_f32<T>(y, row * ldy + col, v + (bias != nullptr ? load_f32<T>(bias, col) : 0.f));
  }
}

// blocks a split-K product aims at: the reduce-kernel form (fp32, direct
// calls) fills the CUs twice; the form whose partials the next kernel adds
// (bf16 prompt forwards) once: 128-token 0.5B TTFT 1.62 ms at 512 blocks,
// 1.49 at 256 (128: 1.53, 192: 1.51, 384: 1.56; per-product mixes of 192-1024
// no better), 512-token 7B 12.67 -> 12.16 ms
#ifndef MINITP_SPLIT_BLOCKS
#define MINITP_SPLIT_BLOCKS 512
#endif
#ifndef MINITP_PARTIALS_SPLIT_BLOCKS
#define MINITP_PARTIALS_SPLIT_BLOCKS 256
#endif
// the same on 128 x 128 tiles (prompts of 512 rows and more): 7B 512-token
// TTFT 11.13 ms at 384 blocks, 11.30 at 320, 11.43-11.46 at 192-256
#ifndef MINITP_PARTIALS_SPLIT_BLOCKS_LARGE
#define MINITP_PARTIALS_SPLIT_BLOCKS_LARGE 384
#endif
// Splits of K (and K elements per split) for an M x N x K product on BM x BN
// tiles: enough blocks to fill the CUs twice, each at least one chunk deep,
// and partials that fit the workspace.
template <typename T, int BM, int BN>
int64_t split_plan(int64_t M, int64_t N, int64_t K, const float* ws, int64_t ws_bytes, int64_t* kper_out,
                   int64_t target = MINITP_SPLIT_BLOCKS) {
  constexpr int64_t KCE = chunk_bytes<BM>() / sizeof(T);
  const int64_t tiles = cdiv(N, BN) * cdiv(M, BM);
  const int64_t nchunk = cdiv(K, KCE);
  int64_t S = 1;
  if (ws != nullptr) {
    S = std::min<int64_t>(cdiv(target, tiles), nchunk);
    while (S > 1 && S * M * N * (int64_t)sizeof(float) > ws_bytes) --S;
  }
  const int64_t kper = cdiv(nchunk, S) * KCE;
  *kper_out = kper;
  return cdiv(K, kper);
}

inline bool gemm_operands_fit(int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t es) {
  return N * K * es <= 0xffffffffLL && ((M - 1) * ldx + K) * es <= 0xffffffffLL;
}

template <typename T, int BM, int BN>
int gemm_launch(hipStream_t st, const T* x, int64_t ldx, const T* w, const T* bias, T* y, int64_t ldy, int64_t M,
                int64_t N, int64_t K, int epi, const T* aux, const StepState* state, float* ws, int64_t ws_bytes) {
  if (!gemm_operands_fit(M, N, K, ldx, sizeof(T))) {
    set_error("gemm: operands over 4 GiB (M=%lld N=%lld K=%lld)", (long long)M, (long long)N, (long long)K);
    return MINITP_ERR_UNSUPPORTED;
  }
  int64_t kper = 0;
  const int64_t S = split_plan<T, BM, BN>(M, N, K, ws, ws_bytes, &kper);
  const dim3 grid((unsigned)cdiv(N, BN), (unsigned)cdiv(M, BM), (unsigned)S);
  if (S > 1) {
    hipLaunchKernelGGL((gemm_kernel<T, BM, BN, OUT_PARTIAL>), grid, dim3(256), 0, st, x, ldx, w, bias, y, ldy, aux,
                       ws, M, N, K, kper, state);
    MINITP_LAUNCH_CHECK();
    const int rgrid = (int)std::min<int64_t>(cdiv(M * N, 256), 2048);
    if (epi == MINITP_EPI_RESID)
      hipLaunchKernelGGL((gemm_reduce_kernel<T, MINITP_EPI_RESID>), dim3(rgrid), dim3(256), 0, st, ws, (int)S, bias,
                         y, ldy, aux, M, N, state);
    else
      hipLaunchKernelGGL((gemm_reduce_kernel<T, MINITP_EPI_NONE>), dim3(rgrid), dim3(256), 0, st, ws, (int)S, bias, y,
                         ldy, aux, M, N, state);
  } else if (epi == MINITP_EPI_RESID) {
    hipLaunchKernelGGL((gemm_kernel<T, BM, BN, MINITP_EPI_RESID>), grid, dim3(256), 0, st, x, ldx, w, bias, y, ldy,
                       aux, ws, M, N, K, kper, state);
  } else {
    hipLaunchKernelGGL((gemm_kernel<T, BM, BN, MINITP_EPI_NONE>), grid, dim3(256), 0, st, x, ldx, w, bias, y, ldy,
                       aux, ws, M, N, K, kper, state);
  }
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

template <typename T>
int gemm_typed(hipStream_t st, const void* x, int64_t ldx, const void* w, const void* bias, void* y, int64_t ldy,
               int64_t M, int64_t N, int64_t K, int epi, const void* aux, const StepState* state, void* ws,
               int64_t ws_bytes) {
  // large M: 128 x 128 tiles already fill the chip; small M: 64 x 64 tiles and split K
  if (M >= 512)
    return gemm_launch<T, 128, 128>(st, (const T*)x, ldx, (const T*)w, (const T*)bias, (T*)y, ldy, M, N, K, epi,
                                    (const T*)aux, state, (float*)ws, ws_bytes);
  return gemm_launch<T, MINITP_GEMM_SMALL_BM, MINITP_GEMM_SMALL_BN>(st, (const T*)x, ldx, (const T*)w,
                                                                    (const T*)bias, (T*)y, ldy, M, N, K, epi,
                                                                    (const T*)aux, state, (float*)ws, ws_bytes);
}

}  // namespace

int launch_gemm_swiglu(hipStream_t st, int dtype, const void* x, int64_t ldx, const void* w, void* y, int64_t ldy,
                       int64_t M, int64_t N, int64_t K) {
  if (M == 0 || N == 0) return MINITP_OK;
  if (dtype != MINITP_BF16 || M >= 512 || ldy < N || !aligned16(x) || !aligned16(w) ||
      !gemm_operands_fit(M, 2 * N, K, ldx, 2)) {
    set_error("gemm: SwiGLU form M=%lld N=%lld K=%lld not served", (long long)M, (long long)N, (long long)K);
    return MINITP_ERR_UNSUPPORTED;
  }
  constexpr int BM = MINITP_GEMM_SMALL_BM, BN = MINITP_GEMM_SMALL_BN;
  const dim3 grid((unsigned)cdiv(N, BN / 2), (unsigned)cdiv(M, BM), 1u);
  hipLaunchKernelGGL((gemm_kernel<bf16, BM, BN, OUT_SWIGLU>), grid, dim3(256), 0, st, (const bf16*)x, ldx,
                     (const bf16*)w, nullptr, (bf16*)y, ldy, nullptr, nullptr, M, N, K, K, nullptr);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

int launch_gemm_partials(hipStream_t st, int dtype, const void* x, int64_t ldx, const void* w, int64_t M, int64_t N,
                         int64_t K, void* ws, int64_t ws_bytes, Partials* out, int64_t target_blocks) {
  if (target_blocks <= 0) target_blocks = M >= 512 ? MINITP_PARTIALS_SPLIT_BLOCKS_LARGE : MINITP_PARTIALS_SPLIT_BLOCKS;
  // the product launch_gemm would split (bf16, not on the tile kernel)
  if (dtype != MINITP_BF16 || M <= 0 || N % 8 != 0 || ws == nullptr || !aligned16(ws) || !aligned16(x) ||
      !aligned16(w) || gemm_tile_supported(M, N, K, ldx, N, false) || !gemm_operands_fit(M, N, K, ldx, 2))
    return MINITP_ERR_UNSUPPORTED;
  int64_t kper = 0, S;
  dim3 grid;
  const bf16 *xb = (const bf16*)x, *wb = (const bf16*)w;
  float* part = (float*)ws;
  if (M >= 512) {
    S = split_plan<bf16, 128, 128>(M, N, K, part, ws_bytes, &kper, target_blocks);
    if (S < 2) return MINITP_ERR_UNSUPPORTED;
    grid = dim3((unsigned)cdiv(N, 128), (unsigned)cdiv(M, 128), (unsigned)S);
    hipLaunchKernelGGL((gemm_kernel<bf16, 128, 128, OUT_PARTIAL>), grid, dim3(256), 0, st, xb, ldx, wb, nullptr,
                       nullptr, N, nullptr, part, M, N, K, kper, nullptr);
  } else {
    constexpr int BM = MINITP_GEMM_SMALL_BM, BN = MINITP_GEMM_SMALL_BN;
    S = split_plan<bf16, BM, BN>(M, N, K, part, ws_bytes, &kper, target_blocks);
    if (S < 2) return MINITP_ERR_UNSUPPORTED;
    grid = dim3((unsigned)cdiv(N, BN), (unsigned)cdiv(M, BM), (unsigned)S);
    hipLaunchKernelGGL((gemm_kernel<bf16, BM, BN, OUT_PARTIAL>), grid, dim3(256), 0, st, xb, ldx, wb, nullptr, nullptr,
                       N, nullptr, part, M, N, K, kper, nullptr);
  }
  MINITP_LAUNCH_CHECK();
  *out = Partials{part, (int)S, M, N};
  return MINITP_OK;
}

int launch_gemm(hipStream_t st, int dtype, const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                int64_t ldy, int64_t M, int64_t N, int64_t K, int epi, const void* aux, const StepState* state,
                void* ws, int64_t ws_bytes, TileTail tail) {
  if (M == 0 || N == 0) return MINITP_OK;
  if (epi != MINITP_EPI_NONE && epi != MINITP_EPI_RESID) {
    set_error("gemm: epilogue %d not supported (split SwiGLU runs as its own kernel)", epi);
    return MINITP_ERR_UNSUPPORTED;
  }
  // bf16 products large enough to fill the chip with 256 x 256 tiles
  if (dtype == MINITP_BF16 && epi == MINITP_EPI_NONE && state == nullptr && aligned16(x) && aligned16(w) &&
      gemm_tile_supported(M, N, K, ldx, ldy, false))
    return launch_gemm_tile(st, x, ldx, w, bias, y, ldy, M, N, K, false, tail);
  return dtype == MINITP_F32 ? gemm_typed<float>(st, x, ldx, w, bias, y, ldy, M, N, K, epi, aux, state, ws, ws_bytes)
                             : gemm_typed<bf16>(st, x, ldx, w, bias, y, ldy, M, N, K, epi, aux, state, ws, ws_bytes);
}

}  // namespace minitp
