// Rotary embedding (rotate_half pairs (i, i + D/2), fp32 tables) and KV writes.
#include "common.h"
#include "kernels.h"

namespace minitp {

// rotate(x)[i]       = x[i] * cos[i]       - x[i+h] * sin[i]
// rotate(x)[i + h]   = x[i+h] * cos[i+h]   + x[i] * sin[i+h]
// with each multiply and the add rounded separately in fp32 (rope.py:61-62).
__device__ __forceinline__ void rotate_pair(float xa, float xb, const float* cr, const float* sr, int i, int half,
                                            float& oa, float& ob) {
  oa = add_rn(mul_rn(xa, cr[i]), -mul_rn(xb, sr[i]));
  ob = add_rn(mul_rn(xb, cr[i + half]), mul_rn(xa, sr[i + half]));
}

// q [B, Hq, T, D], k [B, Hkv, T, D]: one thread per (row, pair).
template <typename T>
__global__ void rope_kernel(const T* q, const T* k, T* q_out, T* k_out, const float* cos_tab, const float* sin_tab,
                            const int64_t* positions, int64_t B, int64_t Hq, int64_t Hkv, int64_t T_, int64_t D) {
  const int64_t half = D / 2;
  const int64_t nq = B * Hq * T_ * half, nk = B * Hkv * T_ * half;
  int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (idx >= nq + nk) return;
  const bool is_q = idx < nq;
  if (!is_q) idx -= nq;
  const int64_t i = idx % half, row = idx / half;  // row = (b, h, t)
  const int64_t t = row % T_;
  const T* src = (is_q ? q : k) + row * D;
  T* dst = (is_q ? q_out : k_out) + row * D;
  const int64_t pos = positions[t];
  float oa, ob;
  rotate_pair(load_f32<T>(src, i), load_f32<T>(src, i + half), cos_tab + pos * D, sin_tab + pos * D, (int)i,
              (int)half, oa, ob);
  store_f32<T>(dst, i, oa);
  store_f32<T>(dst, i + half, ob);
}

int launch_rope(hipStream_t st, int dtype, const void* q, const void* k, void* q_out, void* k_out, const float* cos_tab,
                const float* sin_tab, const int64_t* positions, int64_t B, int64_t Hq, int64_t Hkv, int64_t T_,
                int64_t D) {
  const int64_t n = B * (Hq + Hkv) * T_ * (D / 2);
  if (n == 0) return MINITP_OK;
  const unsigned grid = (unsigned)cdiv(n, 256);
  if (dtype == MINITP_F32)
    rope_kernel<float><<<grid, 256, 0, st>>>((const float*)q, (const float*)k, (float*)q_out, (float*)k_out, cos_tab,
                                             sin_tab, positions, B, Hq, Hkv, T_, D);
  else
    rope_kernel<bf16><<<grid, 256, 0, st>>>((const bf16*)q, (const bf16*)k, (bf16*)q_out, (bf16*)k_out, cos_tab,
                                            sin_tab, positions, B, Hq, Hkv, T_, D);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

// k_new/v_new [B, H, T, D] -> cache [B, H, S, D] rows cache_len + t.
template <typename T>
__global__ void kv_write_kernel(const T* k_new, const T* v_new, T* k_cache, T* v_cache, int64_t B, int64_t H,
                                int64_t T_, int64_t D, int64_t S, int64_t cache_len) {
  const int64_t n = B * H * T_ * D;
  int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (idx >= 2 * n) return;
  const bool is_k = idx < n;
  if (!is_k) idx -= n;
  const int64_t d = idx % D, row = idx / D;
  const int64_t t = row % T_, bh = row / T_;
  const int64_t dst = (bh * S + cache_len + t) * D + d;
  if (is_k)
    k_cache[dst] = k_new[idx];
  else
    v_cache[dst] = v_new[idx];
}

int launch_kv_write(hipStream_t st, int dtype, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                    int64_t B, int64_t H, int64_t T_, int64_t D, int64_t S, int64_t cache_len) {
  const int64_t n = 2 * B * H * T_ * D;
  if (n == 0) return MINITP_OK;
  const unsigned grid = (unsigned)cdiv(n, 256);
  if (dtype == MINITP_F32)
    kv_write_kernel<float><<<grid, 256, 0, st>>>((const float*)k_new, (const float*)v_new, (float*)k_cache,
                                                 (float*)v_cache, B, H, T_, D, S, cache_len);
  else
    kv_write_kernel<bf16><<<grid, 256, 0, st>>>((const bf16*)k_new, (const bf16*)v_new, (bf16*)k_cache,
                                                (bf16*)v_cache, B, H, T_, D, S, cache_len);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

// qkv [B*T, (Hq+2Hkv)*D] -> q_out [B, T, Hq, D] (rotated), k rotated / v
// copied into the caches at cache_len + t. One thread per (token, head, pair).
template <typename T>
__global__ void rope_kv_write_kernel(const T* qkv, int64_t ld, T* q_out, T* k_cache, T* v_cache, const float* cos_tab,
                                     const float* sin_tab, const int64_t* positions, int64_t max_pos, int64_t B,
                                     int64_t T_, int64_t Hq, int64_t Hkv, int64_t D, int64_t S, int64_t cache_len,
                                     int32_t* error_flag, const StepState* state, int layer) {
  if (state != nullptr) {  // graph replay: per-step values live in device memory
    const int64_t layer_off = (int64_t)layer * B * Hkv * S * D;
    positions = state->args.positions;
    cache_len = state->args.cache_len;
    k_cache = (T*)state->args.k_cache + layer_off;
    v_cache = (T*)state->args.v_cache + layer_off;
    error_flag = (int32_t*)&state->error;
  }
  const int64_t half = D / 2, heads = Hq + 2 * Hkv;
  int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (idx >= B * T_ * heads * half) return;
  const int64_t i = idx % half;
  const int64_t head = (idx / half) % heads;
  if (state != nullptr && state->halted && head >= Hq) return;  // early stop reached: no KV rows
  const int64_t n = idx / (half * heads);  // token row b*T + t
  const int64_t b = n / T_, t = n % T_;
  const T* src = qkv + n * ld + head * D;
  const float xa = load_f32<T>(src, i), xb = load_f32<T>(src, i + half);
  if (head < Hq + Hkv) {
    const int64_t pos = positions[t];
    float oa, ob;
    if (pos < 0 || pos >= max_pos) {
      oa = ob = __builtin_nanf("");
      if (error_flag) *error_flag = 1;
    } else {
      rotate_pair(xa, xb, cos_tab + pos * D, sin_tab + pos * D, (int)i, (int)half, oa, ob);
    }
    T* dst = head < Hq ? q_out + (n * Hq + head) * D
                       : k_cache + ((b * Hkv + (head - Hq)) * S + cache_len + t) * D;
    store_f32<T>(dst, i, oa);
    store_f32<T>(dst, i + half, ob);
  } else {
    T* dst = v_cache + ((b * Hkv + (head - Hq - Hkv)) * S + cache_len + t) * D;
    store_f32<T>(dst, i, xa);
    store_f32<T>(dst, i + half, xb);
  }
}

int launch_rope_kv_write(hipStream_t st, int dtype, const void* qkv, int64_t ld_qkv, void* q_out, void* k_cache,
                         void* v_cache, const float* cos_tab, const float* sin_tab, const int64_t* positions,
                         int64_t max_pos, int64_t B, int64_t T_, int64_t Hq, int64_t Hkv, int64_t D, int64_t S,
                         int64_t cache_len, int32_t* error_flag, const StepState* state, int layer) {
  const int64_t n = B * T_ * (Hq + 2 * Hkv) * (D / 2);
  if (n == 0) return MINITP_OK;
  const unsigned grid = (unsigned)cdiv(n, 256);
  if (dtype == MINITP_F32)
    rope_kv_write_kernel<float><<<grid, 256, 0, st>>>((const float*)qkv, ld_qkv, (float*)q_out, (float*)k_cache,
                                                      (float*)v_cache, cos_tab, sin_tab, positions, max_pos, B, T_,
                                                      Hq, Hkv, D, S, cache_len, error_flag, state, layer);
  else
    rope_kv_write_kernel<bf16><<<grid, 256, 0, st>>>((const bf16*)qkv, ld_qkv, (bf16*)q_out, (bf16*)k_cache,
                                                     (bf16*)v_cache, cos_tab, sin_tab, positions, max_pos, B, T_, Hq,
                                                     Hkv, D, S, cache_len, error_flag, state, layer);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

}  // namespace minitp
