// Greedy selection over a logits row (embedding.py:146-147, generation.py:59).
// torch.argmax order: the first maximum wins; a NaN beats every number.
// Grid (slices, rows): each block reduces one slice of a row to a (value,
// index) partial; a one-block-per-row kernel merges the partials.
#include <mutex>

#include "common.h"
#include "kernels.h"

// Slice partials of minitp_argmax_static, the allocation-free argmax: one
// array per device, held until the process ends. Host code never passes
// `scratch` itself to a kernel (on the host it is only a stand-in symbol);
// it passes the device address hipGetSymbolAddress returns for the device.
constexpr int64_t ARGMAX_SCRATCH_BYTES = 1 << 20;
static __device__ __align__(256) unsigned char scratch[ARGMAX_SCRATCH_BYTES];

namespace minitp {

namespace {

constexpr int SLICE = 256 * 16;  // elements per block

// Block partial of one slice of a row: (value, index) into pv / pi [row][nb].
template <typename T>
__global__ __launch_bounds__(256) void argmax_slice_kernel(const T* logits, int64_t ld, int64_t V, float* pv,
                                                           int64_t* pi, const StepState* state, int64_t row_offset) {
  if (state != nullptr) logits = (const T*)state->args.logits + row_offset;
  __shared__ float wv[4];
  __shared__ int64_t wi[4];
  const int64_t row = blockIdx.y, nb = gridDim.x;
  const T* lr = logits + row * ld;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float v = -__builtin_inff();
  int64_t i = INT64_MAX;
  const int64_t start = (int64_t)blockIdx.x * SLICE, end = std::min<int64_t>(V, start + SLICE);
  if ((((uint64_t)lr) & 15) == 0 && V * (int64_t)sizeof(T) < (1LL << 31)) {
    // 16 consecutive elements per thread, every 16-byte load issued before
    // the first comparison. Only whole vectors inside the row are loaded
    // that way (the others read zeros and are dropped by index); a vector
    // that straddles the row's end is read element by element below.
    constexpr int VE = 16 / (int)sizeof(T), NV = 16 / VE;
    const __amdgpu_buffer_rsrc_t r = span_rsrc(lr, (uint32_t)(V * (int64_t)sizeof(T)));
    const int64_t j0 = start + 16 * tid;
    uint4 raw[NV];
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int64_t j = j0 + u * VE;
      const u32x4 w = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     r, j + VE <= end ? (uint32_t)(j * (int64_t)sizeof(T)) : 0xffffffffu, 0, 0));
      raw[u] = make_uint4(w.x, w.y, w.z, w.w);
    }
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int64_t j = j0 + u * VE;
      if (j < end && j + VE > end) {  // the straddling vector: its elements one by one
        for (int64_t e = j; e < end; ++e) {
          const float x = load_f32<T>(lr, e);
          if (argmax_better(x, e, v, i)) {
            v = x;
            i = e;
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const uint32_t wd[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        const int64_t j = j0 + u * VE + e;
        float x;
        if constexpr (sizeof(T) == 2)
          x = bf16_to_f32((uint16_t)(wd[e / 2] >> (16 * (e % 2))));
        else
          x = __builtin_bit_cast(float, wd[e]);
        if (j0 + u * VE + VE <= end && argmax_better(x, j, v, i)) {
          v = x;
          i = j;
        }
      }
    }
  } else {
    for (int64_t j = start + tid; j < end; j += 256) {
      const float x = load_f32<T>(lr, j);
      if (argmax_better(x, j, v, i)) {
        v = x;
        i = j;
      }
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
  }
}

// Winner of each row's nb partials (block = row). A separate launch: the
// partials of the previous kernel are visible without a grid-wide fence,
// which on a multi-XCD part writes back and invalidates L2 per block.
__global__ __launch_bounds__(256) void argmax_merge_kernel(const float* pv, const int64_t* pi, int64_t nb,
                                                           int64_t* out, int64_t out_stride, const StepState* state) {
  if (state != nullptr) {
    out = state->args.next_tok;
    out_stride = state->args.next_tok_ld;
  }
  __shared__ float wv[4];
  __shared__ int64_t wi[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float v = -__builtin_inff();
  int64_t i = INT64_MAX;
  // partials in batches of four per thread, every load of a batch issued
  // before the first comparison (a loop that compares as it loads waits one
  // memory round trip per partial)
  for (int64_t j0 = tid; j0 < nb; j0 += 4 * 256) {
    float x[4];
    int64_t xi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int64_t j = j0 + 256 * k;
      const int64_t jj = j < nb ? j : j0;  // in bounds; dropped below
      x[k] = pv[row * nb + jj];
      xi[k] = pi[row * nb + jj];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (j0 + 256 * k < nb && argmax_better(x[k], xi[k], v, i)) {
        v = x[k];
        i = xi[k];
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
    if (out != nullptr) out[row * out_stride] = i;
  }
}

int64_t nslices(int64_t V) { return std::max<int64_t>(1, cdiv(V, SLICE)); }

// generate_greedy's finished mask (generation.py:153-168) after a token
// selection: tok = finished ? eos : tok; finished |= tok == eos. Once every
// row has finished, the halted word and the stop column are set (and the
// stop column stored to the host word); a forward that starts halted leaves
// tokens and flags alone.
__global__ __launch_bounds__(256) void eos_update_kernel(const StepState* state, int64_t B) {
  const StepArgs& a = state->args;
  int64_t* es = a.eos_state;
  if (es == nullptr || es[B] != 0) return;  // the same answer for every thread
  __shared__ int unfinished;
  if (threadIdx.x == 0) unfinished = 0;
  __syncthreads();
  for (int64_t b = threadIdx.x; b < B; b += blockDim.x) {
    int64_t* slot = a.next_tok + b * a.next_tok_ld;
    const bool was = es[b] != 0;
    if (was) *slot = a.eos_token;
    const bool fin = was || *slot == a.eos_token;
    es[b] = fin ? 1 : 0;
    if (!fin) unfinished = 1;
  }
  __syncthreads();
  if (threadIdx.x == 0 && unfinished == 0) {
    es[B] = 1;
    es[B + 1] = a.cursor + 1;
    if (a.eos_host != nullptr)
      __hip_atomic_store(a.eos_host, a.cursor + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

}  // namespace

int launch_eos_update(hipStream_t st, const StepState* state, int64_t B) {
  eos_update_kernel<<<1, 256, 0, st>>>(state, B);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

int64_t argmax_workspace_bytes(int64_t B, int64_t V) { return B * nslices(V) * (4 + 8); }

int launch_argmax_merge(hipStream_t st, const float* pv, const int64_t* pi, int64_t nb, int64_t rows, int64_t* out,
                        int64_t out_stride, const StepState* state) {
  if (rows == 0) return MINITP_OK;
  argmax_merge_kernel<<<(unsigned)rows, 256, 0, st>>>(pv, pi, nb, out, out_stride, state);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

namespace {

constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_ptr[SCRATCH_MAX_DEVICES];  // device address of `scratch`, per device

// Device address of `scratch` on `dev`, looked up once per device with that
// device current (each device holds its own copy at its own address).
int scratch_address(int dev, void** out) {
  if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) {
    set_error("argmax_static: device %d beyond the %d this library tracks", dev, SCRATCH_MAX_DEVICES);
    return MINITP_ERR_ARG;
  }
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_ptr[dev] == nullptr) {
    int cur = 0;
    MINITP_RETURN_HIP(hipGetDevice(&cur));
    if (cur != dev) MINITP_RETURN_HIP(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) MINITP_RETURN_HIP(hipSetDevice(cur));
    MINITP_RETURN_HIP(e);
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return MINITP_OK;
}

}  // namespace

int64_t argmax_static_scratch_bytes() { return ARGMAX_SCRATCH_BYTES; }

int launch_argmax_static(hipStream_t st, int dtype, const void* logits, int64_t ld, int64_t B, int64_t V, int64_t* out,
                         int64_t out_stride) {
  if (B == 0) return MINITP_OK;
  const int64_t need = argmax_workspace_bytes(B, V);
  if (need > ARGMAX_SCRATCH_BYTES) {
    set_error("argmax_static: %lld rows x %lld slices need %lld B of partials, more than the %lld B static scratch "
              "(use minitp_argmax with a workspace)",
              (long long)B, (long long)nslices(V), (long long)need, (long long)ARGMAX_SCRATCH_BYTES);
    return MINITP_ERR_ARG;
  }
  int dev = 0;
  if (st != nullptr) {
    hipDevice_t d = 0;
    MINITP_RETURN_HIP(hipStreamGetDevice(st, &d));
    dev = (int)d;
  } else {
    MINITP_RETURN_HIP(hipGetDevice(&dev));
  }
  void* ws = nullptr;
  if (const int rc = scratch_address(dev, &ws)) return rc;
  // every partial the merge reads is written by the slice kernel first:
  // nothing in the scratch has to start at zero
  return launch_argmax(st, dtype, logits, ld, B, V, out, out_stride, ws, need, nullptr, 0);
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
  int64_t* pi = (int64_t*)workspace;
  float* pv = (float*)(pi + B * nb);
  dim3 grid((unsigned)nb, (unsigned)B);
  if (dtype == MINITP_F32)
    argmax_slice_kernel<float><<<grid, 256, 0, st>>>((const float*)logits, ld, V, pv, pi, state, row_offset);
  else
    argmax_slice_kernel<bf16><<<grid, 256, 0, st>>>((const bf16*)logits, ld, V, pv, pi, state, row_offset);
  MINITP_LAUNCH_CHECK();
  return launch_argmax_merge(st, pv, pi, nb, B, out, out_stride, state);
}

}  // namespace minitp
