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

__device__ __forceinline__ void store8_bf16(bf16* dst, const float* v) {
  if (((uintptr_t)dst & 15u) == 0) {
    *reinterpret_cast<uint4*>(dst) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) store_f32<bf16>(dst, e, v[e]);
  }
}

// The same as rope_kv_write_kernel<bf16> for D / 2 % 8 == 0, eight pairs per
// thread: 16-byte loads of the qkv row (the caller checks its alignment) and
// of the fp32 tables, 16-byte stores wherever the destination allows them.
// PART: the projection is the split-K partial product (qp) plus the bias,
// rounded to bf16 as gemm_reduce_kernel stores it, instead of a qkv row.
template <bool PART>
__global__ void rope_kv_write8_kernel(const bf16* qkv, int64_t ld, Partials qp, const bf16* bias, bf16* q_out,
                                      bf16* k_cache, bf16* v_cache, const float* cos_tab, const float* sin_tab,
                                      const int64_t* positions, int64_t max_pos, int64_t B, int64_t T_, int64_t Hq,
                                      int64_t Hkv, int64_t D, int64_t S, int64_t cache_len, int32_t* error_flag,
                                      const StepState* state, int layer) {
  if (state != nullptr) {
    const int64_t layer_off = (int64_t)layer * B * Hkv * S * D;
    positions = state->args.positions;
    cache_len = state->args.cache_len;
    k_cache = (bf16*)state->args.k_cache + layer_off;
    v_cache = (bf16*)state->args.v_cache + layer_off;
    error_flag = (int32_t*)&state->error;
  }
  const int64_t half = D / 2, groups = half / 8, heads = Hq + 2 * Hkv;
  int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (idx >= B * T_ * heads * groups) return;
  const int64_t i = (idx % groups) * 8;
  const int64_t head = (idx / groups) % heads;
  if (state != nullptr && state->halted && head >= Hq) return;
  const int64_t n = idx / (groups * heads);
  const int64_t b = n / T_, t = n % T_;
  float xa[8], xb[8], oa[8], ob[8];
  if constexpr (PART) {
    const int64_t col = head * D + i;
    float va[8], vb[8], ba[8], bb[8];
    sum_partials8(qp, n, col, va);
    sum_partials8(qp, n, col + half, vb);
    unpack16(*reinterpret_cast<const uint4*>(bias + col), ba, (bf16*)nullptr);
    unpack16(*reinterpret_cast<const uint4*>(bias + col + half), bb, (bf16*)nullptr);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xa[e] = round_to<bf16>(va[e] + ba[e]);
      xb[e] = round_to<bf16>(vb[e] + bb[e]);
    }
  } else {
    const bf16* src = qkv + n * ld + head * D;
    unpack16(*reinterpret_cast<const uint4*>(src + i), xa, (bf16*)nullptr);
    unpack16(*reinterpret_cast<const uint4*>(src + i + half), xb, (bf16*)nullptr);
  }
  bf16* dst;
  if (head < Hq + Hkv) {
    const int64_t pos = positions[t];
    if (pos < 0 || pos >= max_pos) {
#pragma unroll
      for (int e = 0; e < 8; ++e) oa[e] = ob[e] = __builtin_nanf("");
      if (error_flag) *error_flag = 1;
    } else {
      const float4* cr = reinterpret_cast<const float4*>(cos_tab + pos * D + i);
      const float4* sr = reinterpret_cast<const float4*>(sin_tab + pos * D + i);
      const float4 c0 = cr[0], c1 = cr[1], s0 = sr[0], s1 = sr[1];
      const float4 c2 = cr[half / 4], c3 = cr[half / 4 + 1], s2 = sr[half / 4], s3 = sr[half / 4 + 1];
      const float ca[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
      const float sa[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
      const float cb[8] = {c2.x, c2.y, c2.z, c2.w, c3.x, c3.y, c3.z, c3.w};
      const float sb[8] = {s2.x, s2.y, s2.z, s2.w, s3.x, s3.y, s3.z, s3.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        oa[e] = add_rn(mul_rn(xa[e], ca[e]), -mul_rn(xb[e], sa[e]));
        ob[e] = add_rn(mul_rn(xb[e], cb[e]), mul_rn(xa[e], sb[e]));
      }
    }
    dst = head < Hq ? q_out + (n * Hq + head) * D : k_cache + ((b * Hkv + (head - Hq)) * S + cache_len + t) * D;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      oa[e] = xa[e];
      ob[e] = xb[e];
    }
    dst = v_cache + ((b * Hkv + (head - Hq - Hkv)) * S + cache_len + t) * D;
  }
  store8_bf16(dst + i, oa);
  store8_bf16(dst + i + half, ob);
}

int launch_rope_kv_write(hipStream_t st, int dtype, const void* qkv, int64_t ld_qkv, void* q_out, void* k_cache,
                         void* v_cache, const float* cos_tab, const float* sin_tab, const int64_t* positions,
                         int64_t max_pos, int64_t B, int64_t T_, int64_t Hq, int64_t Hkv, int64_t D, int64_t S,
                         int64_t cache_len, int32_t* error_flag, const StepState* state, int layer) {
  const int64_t n = B * T_ * (Hq + 2 * Hkv) * (D / 2);
  if (n == 0) return MINITP_OK;
  if (dtype == MINITP_BF16 && D % 16 == 0 && ld_qkv % 8 == 0 && aligned16(qkv) && aligned16(cos_tab) &&
      aligned16(sin_tab)) {
    rope_kv_write8_kernel<false><<<(unsigned)cdiv(n / 8, 256), 256, 0, st>>>(
        (const bf16*)qkv, ld_qkv, Partials{}, nullptr, (bf16*)q_out, (bf16*)k_cache, (bf16*)v_cache, cos_tab, sin_tab,
        positions, max_pos, B, T_, Hq, Hkv, D, S, cache_len, error_flag, state, layer);
    MINITP_LAUNCH_CHECK();
    return MINITP_OK;
  }
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

int launch_rope_kv_write_partials(hipStream_t st, const Partials& qkv, const void* bias, void* q_out,
                                  const float* cos_tab, const float* sin_tab, int64_t max_pos, int64_t B, int64_t T_,
                                  int64_t Hq, int64_t Hkv, int64_t D, int64_t S, const StepState* state, int layer) {
  const int64_t n = B * T_ * (Hq + 2 * Hkv) * (D / 2);
  if (n == 0) return MINITP_OK;
  if (state == nullptr || bias == nullptr || D % 16 != 0 || qkv.M != B * T_ || qkv.N != (Hq + 2 * Hkv) * D ||
      qkv.S < 1 || !aligned16(qkv.p) || !aligned16(bias) || !aligned16(cos_tab) || !aligned16(sin_tab)) {
    set_error("rope_kv_write from partials: D %lld, partial width %lld", (long long)D, (long long)qkv.N);
    return MINITP_ERR_UNSUPPORTED;
  }
  rope_kv_write8_kernel<true><<<(unsigned)cdiv(n / 8, 256), 256, 0, st>>>(
      nullptr, 0, qkv, (const bf16*)bias, (bf16*)q_out, nullptr, nullptr, cos_tab, sin_tab, nullptr, max_pos, B, T_, Hq,
      Hkv, D, S, 0, nullptr, state, layer);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

}  // namespace minitp
