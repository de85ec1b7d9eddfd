// Greedy selection over a logits row (embedding.py:146-147, generation.py:59).
// torch.argmax order: the first maximum wins; a NaN beats every number.
// Grid (slices, rows): each block reduces one slice of a row, writes a
// (value, index) partial, and the last block of the row merges them.
#include "common.h"
#include "kernels.h"

namespace minitp {

namespace {

constexpr int SLICE = 256 * 16;  // elements per block

template <typename T>
__global__ __launch_bounds__(256) void argmax_kernel(const T* logits, int64_t ld, int64_t V, int64_t* out,
                                                     int64_t out_stride, unsigned* counters, float* pv, int64_t* pi,
                                                     const StepState* state, int64_t row_offset) {
  if (state != nullptr) {
    logits = (const T*)state->logits + row_offset;
    out = state->next_tok;
    out_stride = state->next_tok_ld;
  }
  __shared__ float wv[4];
  __shared__ int64_t wi[4];
  __shared__ bool last_block;
  const int64_t row = blockIdx.y, nb = gridDim.x;
  const T* lr = logits + row * ld;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float v = -__builtin_inff();
  int64_t i = INT64_MAX;
  const int64_t end = std::min<int64_t>(V, ((int64_t)blockIdx.x + 1) * SLICE);
  for (int64_t j = (int64_t)blockIdx.x * SLICE + tid; j < end; j += 256) {
    const float x = load_f32<T>(lr, j);
    if (argmax_better(x, j, v, i)) {
      v = x;
      i = j;
    }
  }
  wave_argmax(v, i);
  if (lane == 0) {
    wv[wave] = v;
    wi[wave] = i;
  }
  __syncthreads();
  if (tid == 0) {
    for (int s = 1; s < 4; ++s)
      if (argmax_better(wv[s], wi[s], v, i)) {
        v = wv[s];
        i = wi[s];
      }
    pv[row * nb + blockIdx.x] = v;
    pi[row * nb + blockIdx.x] = i;
    __threadfence();
    last_block = atomicAdd(&counters[row], 1u) == (unsigned)nb - 1;
  }
  __syncthreads();
  if (!last_block) return;
  __threadfence();
  v = -__builtin_inff();
  i = INT64_MAX;
  for (int64_t j = tid; j < nb; j += 256) {
    const float x = __hip_atomic_load(&pv[row * nb + j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int64_t xi = __hip_atomic_load(&pi[row * nb + j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (argmax_better(x, xi, v, i)) {
      v = x;
      i = xi;
    }
  }
  wave_argmax(v, i);
  __syncthreads();
  if (lane == 0) {
    wv[wave] = v;
    wi[wave] = i;
  }
  __syncthreads();
  if (tid == 0) {
    for (int s = 1; s < 4; ++s)
      if (argmax_better(wv[s], wi[s], v, i)) {
        v = wv[s];
        i = wi[s];
      }
    if (out != nullptr) out[row * out_stride] = i;
    counters[row] = 0u;
  }
}

int64_t nslices(int64_t V) { return std::max<int64_t>(1, cdiv(V, SLICE)); }

}  // namespace

int64_t argmax_workspace_bytes(int64_t B, int64_t V) {
  return cdiv(B * 4, 256) * 256 + B * nslices(V) * (4 + 8);
}

int launch_argmax(hipStream_t st, int dtype, const void* logits, int64_t ld, int64_t B, int64_t V, int64_t* out,
                  int64_t out_stride, void* workspace, int64_t workspace_bytes, const StepState* state,
                  int64_t row_offset) {
  if (B == 0) return MINITP_OK;
  if (V <= 0) {
    set_error("argmax: empty vocab");
    return MINITP_ERR_ARG;
  }
  if (workspace == nullptr || workspace_bytes < argmax_workspace_bytes(B, V)) {
    set_error("argmax: workspace too small");
    return MINITP_ERR_ARG;
  }
  const int64_t nb = nslices(V);
  char* ws = (char*)workspace;
  unsigned* counters = (unsigned*)ws;
  ws += cdiv(B * 4, 256) * 256;
  int64_t* pi = (int64_t*)ws;
  ws += B * nb * 8;
  float* pv = (float*)ws;
  dim3 grid((unsigned)nb, (unsigned)B);
  if (dtype == MINITP_F32)
    argmax_kernel<float><<<grid, 256, 0, st>>>((const float*)logits, ld, V, out, out_stride, counters, pv, pi,
                                                 state, row_offset);
  else
    argmax_kernel<bf16><<<grid, 256, 0, st>>>((const bf16*)logits, ld, V, out, out_stride, counters, pv, pi,
                                                state, row_offset);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

}  // namespace minitp
