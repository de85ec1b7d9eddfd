// GQA attention over the KV cache (attention.py:77-105 at tp_size == 1).
//
// Q head h reads KV head h / G (G = Hq / Hkv), the order repeat_interleave
// gives (attention.py:89-90), so no K/V copy is ever made. Scale 1/sqrt(D)
// (SDPA default). Softmax and accumulation in fp32; the output is rounded to
// the model dtype once.
#include "common.h"
#include "kernels.h"

namespace minitp {

namespace {

constexpr int CHUNK = 256;  // decode: key positions per block (one per thread)
constexpr int GMAX = 8;     // max q heads per KV head served

struct DecodeArgs {
  const void* q;  // [B, Hq, D] (T == 1)
  const void* k;  // layer base [B, Hkv, S, D] (ignored when st != null)
  const void* v;
  void* out;  // [B, Hq * D]
  AttnShape s;
  int64_t cache_len;
  const StepState* st;
  int layer;
  float scale;
  unsigned* counters;  // [B * Hkv]
  float* ws_ml;        // [B * Hkv][nsplit][GMAX][2]
  float* ws_o;         // [B * Hkv][nsplit][GMAX][D]
  int nsplit_cap;
};

template <typename T, int D>
__global__ __launch_bounds__(256) void decode_attn_kernel(DecodeArgs a) {
  constexpr int NPART = 256 / D;
  __shared__ float qs[GMAX][D];
  __shared__ float ps[GMAX][CHUNK];
  __shared__ float stat[GMAX][2];  // max, sum
  __shared__ float part[NPART > 1 ? NPART : 1][GMAX][D];
  __shared__ bool last_block;

  const AttnShape& s = a.s;
  const int G = s.Hq / s.Hkv;
  const int bh = blockIdx.x, b = bh / s.Hkv, g = bh % s.Hkv;
  const int64_t cache_len = a.st ? a.st->cache_len : a.cache_len;
  const int64_t ctx = cache_len + 1;
  const int64_t j0 = (int64_t)blockIdx.y * CHUNK;
  if (j0 >= ctx) return;  // split beyond the filled cache (block-uniform)
  const int64_t j1 = std::min<int64_t>(j0 + CHUNK, ctx);
  const int nsplit = (int)cdiv(ctx, CHUNK);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  const int64_t layer_off = (int64_t)a.layer * s.B * s.Hkv * s.S * D;
  const T* kc = (const T*)(a.st ? a.st->k_cache : a.k) + (a.st ? layer_off : 0) + (int64_t)bh * s.S * D;
  const T* vc = (const T*)(a.st ? a.st->v_cache : a.v) + (a.st ? layer_off : 0) + (int64_t)bh * s.S * D;
  const T* q = (const T*)a.q;

  for (int i = tid; i < GMAX * D; i += 256) {
    const int gi = i / D, d = i % D;
    qs[gi][d] = gi < G ? load_f32<T>(q, ((int64_t)b * s.Hq + g * G + gi) * D + d) : 0.f;
  }
  __syncthreads();

  // scores: one key row per thread
  {
    float sc[GMAX];
#pragma unroll
    for (int gi = 0; gi < GMAX; ++gi) sc[gi] = 0.f;
    const int64_t j = j0 + tid;
    if (j < j1) {
      constexpr int V = Vec<T>::N;
      const uint4* kr = reinterpret_cast<const uint4*>(kc + j * D);
#pragma unroll
      for (int c = 0; c < D / V; ++c) {
        float kf[V];
        unpack16(kr[c], kf, (T*)nullptr);
#pragma unroll
        for (int gi = 0; gi < GMAX; ++gi)
#pragma unroll
          for (int e = 0; e < V; ++e) sc[gi] = fmaf(qs[gi][c * V + e], kf[e], sc[gi]);
      }
    }
#pragma unroll
    for (int gi = 0; gi < GMAX; ++gi) ps[gi][tid] = j < j1 ? sc[gi] * a.scale : -__builtin_inff();
  }
  __syncthreads();

  // softmax statistics per head over this chunk (wave w takes heads w, w+4)
  for (int gi = wave; gi < G; gi += 4) {
    float mx = -__builtin_inff();
    for (int i = lane; i < CHUNK; i += 64) mx = fmaxf(mx, ps[gi][i]);
    mx = wave_max(mx);
    float sum = 0.f;
    for (int i = lane; i < CHUNK; i += 64) {
      const float p = expf(ps[gi][i] - mx);
      ps[gi][i] = p;
      sum += p;
    }
    sum = wave_sum(sum);
    if (lane == 0) {
      stat[gi][0] = mx;
      stat[gi][1] = sum;
    }
  }
  __syncthreads();

  // P V: thread = (part, d); part p sums keys p, p + NPART, ...
  {
    const int d = tid % D, p = tid / D;
    float acc[GMAX];
#pragma unroll
    for (int gi = 0; gi < GMAX; ++gi) acc[gi] = 0.f;
    if (p < NPART) {
      for (int64_t jj = p; jj < j1 - j0; jj += NPART) {
        const float vv = load_f32<T>(vc, (j0 + jj) * D + d);
#pragma unroll
        for (int gi = 0; gi < GMAX; ++gi) acc[gi] = fmaf(ps[gi][jj], vv, acc[gi]);
      }
#pragma unroll
      for (int gi = 0; gi < GMAX; ++gi) part[p][gi][d] = acc[gi];
    }
  }
  __syncthreads();

  T* out = (T*)a.out;
  if (nsplit == 1) {
    for (int i = tid; i < G * D; i += 256) {
      const int gi = i / D, d = i % D;
      float o = 0.f;
      for (int p = 0; p < NPART; ++p) o += part[p][gi][d];
      store_f32<T>(out, ((int64_t)b * s.Hq + g * G + gi) * D + d, o / stat[gi][1]);
    }
    return;
  }

  // split-K: publish partials; the last split of this (b, kv head) merges
  const int64_t slot = (int64_t)bh * a.nsplit_cap + blockIdx.y;
  for (int i = tid; i < G * D; i += 256) {
    const int gi = i / D, d = i % D;
    float o = 0.f;
    for (int p = 0; p < NPART; ++p) o += part[p][gi][d];
    a.ws_o[(slot * GMAX + gi) * D + d] = o;
  }
  if (tid < G) {
    a.ws_ml[(slot * GMAX + tid) * 2 + 0] = stat[tid][0];
    a.ws_ml[(slot * GMAX + tid) * 2 + 1] = stat[tid][1];
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = atomicAdd(&a.counters[bh], 1u);
    last_block = prev == (unsigned)nsplit - 1;
  }
  __syncthreads();
  if (!last_block) return;
  __threadfence();
  for (int i = tid; i < G * D; i += 256) {
    const int gi = i / D, d = i % D;
    const int64_t base = (int64_t)bh * a.nsplit_cap;
    float mx = -__builtin_inff();
    for (int sp = 0; sp < nsplit; ++sp)
      mx = fmaxf(mx, __hip_atomic_load(&a.ws_ml[((base + sp) * GMAX + gi) * 2], __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT));
    float l = 0.f, o = 0.f;
    for (int sp = 0; sp < nsplit; ++sp) {
      const float m_s = __hip_atomic_load(&a.ws_ml[((base + sp) * GMAX + gi) * 2], __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
      const float l_s = __hip_atomic_load(&a.ws_ml[((base + sp) * GMAX + gi) * 2 + 1], __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
      const float o_s = __hip_atomic_load(&a.ws_o[((base + sp) * GMAX + gi) * D + d], __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
      const float w = expf(m_s - mx);
      l = fmaf(w, l_s, l);
      o = fmaf(w, o_s, o);
    }
    store_f32<T>(out, ((int64_t)b * s.Hq + g * G + gi) * D + d, o / l);
  }
  if (tid == 0) a.counters[bh] = 0u;
}

// ---------------------------------------------------------------------------
// Prefill: flash-style causal attention, fp32 FMA. Block = (b * Hq + h,
// 64-query tile); 4 lanes per query, each owning D/4 dims; key tiles of K
// and V (64 keys, 32 at D = 128) staged in LDS as fp32.
constexpr int QT = 64;

template <typename T, int D>
__global__ __launch_bounds__(256) void prefill_attn_kernel(const T* q, const T* kc, const T* vc, T* out, AttnShape s,
                                                           int64_t cache_len, float scale) {
  constexpr int DQ = D / 4;
  constexpr int KT = D >= 128 ? 32 : 64;
  __shared__ float Ks[KT][D + 1];
  __shared__ float Vs[KT][D + 1];
  const int G = s.Hq / s.Hkv;
  const int bh = blockIdx.x, b = bh / s.Hq, h = bh % s.Hq, g = h / G;
  const int tid = threadIdx.x, qi = tid / 4, quarter = tid % 4;
  const int64_t t = (int64_t)blockIdx.y * QT + qi;  // query index in this forward
  const bool q_ok = t < s.T;
  const T* kbase = kc + ((int64_t)b * s.Hkv + g) * s.S * D;
  const T* vbase = vc + ((int64_t)b * s.Hkv + g) * s.S * D;

  float qv[DQ], o[DQ];
#pragma unroll
  for (int i = 0; i < DQ; ++i) {
    qv[i] = q_ok ? load_f32<T>(q, (((int64_t)b * s.T + t) * s.Hq + h) * D + quarter * DQ + i) : 0.f;
    o[i] = 0.f;
  }
  float m = -__builtin_inff(), l = 0.f;
  const int64_t limit = cache_len + t;  // last key this query may see
  const int64_t t_last = std::min<int64_t>((int64_t)blockIdx.y * QT + QT, s.T) - 1;
  const int64_t key_end = cache_len + t_last + 1;  // keys needed by the tile

  for (int64_t k0 = 0; k0 < key_end; k0 += KT) {
    __syncthreads();
    for (int i = tid; i < KT * D; i += 256) {
      const int j = i / D, d = i % D;
      const bool ok = k0 + j < key_end;
      Ks[j][d] = ok ? load_f32<T>(kbase, (k0 + j) * D + d) : 0.f;
      Vs[j][d] = ok ? load_f32<T>(vbase, (k0 + j) * D + d) : 0.f;
    }
    __syncthreads();
    float sc[KT];
    float tile_max = -__builtin_inff();
#pragma unroll 8
    for (int j = 0; j < KT; ++j) {
      float p = 0.f;
#pragma unroll
      for (int i = 0; i < DQ; ++i) p = fmaf(qv[i], Ks[j][quarter * DQ + i], p);
      p += __shfl_xor(p, 1, 64);
      p += __shfl_xor(p, 2, 64);
      const bool ok = k0 + j <= limit;
      sc[j] = ok ? p * scale : -__builtin_inff();
      tile_max = fmaxf(tile_max, sc[j]);
    }
    const float m_new = fmaxf(m, tile_max);
    if (m_new == -__builtin_inff()) continue;  // nothing visible yet
    const float alpha = expf(m - m_new);
    l *= alpha;
#pragma unroll
    for (int i = 0; i < DQ; ++i) o[i] *= alpha;
#pragma unroll 8
    for (int j = 0; j < KT; ++j) {
      const float p = expf(sc[j] - m_new);
      l += p;
#pragma unroll
      for (int i = 0; i < DQ; ++i) o[i] = fmaf(p, Vs[j][quarter * DQ + i], o[i]);
    }
    m = m_new;
  }
  if (q_ok) {
#pragma unroll
    for (int i = 0; i < DQ; ++i)
      store_f32<T>(out, (((int64_t)b * s.T + t) * s.Hq + h) * D + quarter * DQ + i, o[i] / l);
  }
}

template <typename T, int D>
int decode_dispatch(hipStream_t st, DecodeArgs& a, int64_t max_ctx) {
  const int nsplit = (int)cdiv(max_ctx, CHUNK);
  hipLaunchKernelGGL((decode_attn_kernel<T, D>), dim3(a.s.B * a.s.Hkv, nsplit), dim3(256), 0, st, a);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

template <typename T>
int decode_by_d(hipStream_t st, DecodeArgs& a, int64_t max_ctx) {
  switch (a.s.D) {
    case 16:
      return decode_dispatch<T, 16>(st, a, max_ctx);
    case 32:
      return decode_dispatch<T, 32>(st, a, max_ctx);
    case 64:
      return decode_dispatch<T, 64>(st, a, max_ctx);
    case 128:
      return decode_dispatch<T, 128>(st, a, max_ctx);
  }
  set_error("attention: head_dim %d not supported (16, 32, 64, 128)", a.s.D);
  return MINITP_ERR_UNSUPPORTED;
}

template <typename T, int D>
int prefill_dispatch(hipStream_t st, const void* q, const void* k, const void* v, void* out, const AttnShape& s,
                     int64_t cache_len) {
  const float scale = 1.0f / sqrtf((float)D);
  hipLaunchKernelGGL((prefill_attn_kernel<T, D>), dim3(s.B * s.Hq, (unsigned)cdiv(s.T, QT)), dim3(256), 0, st,
                     (const T*)q, (const T*)k, (const T*)v, (T*)out, s, cache_len, scale);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

template <typename T>
int prefill_by_d(hipStream_t st, const void* q, const void* k, const void* v, void* out, const AttnShape& s,
                 int64_t cache_len) {
  switch (s.D) {
    case 16:
      return prefill_dispatch<T, 16>(st, q, k, v, out, s, cache_len);
    case 32:
      return prefill_dispatch<T, 32>(st, q, k, v, out, s, cache_len);
    case 64:
      return prefill_dispatch<T, 64>(st, q, k, v, out, s, cache_len);
    case 128:
      return prefill_dispatch<T, 128>(st, q, k, v, out, s, cache_len);
  }
  set_error("attention: head_dim %d not supported (16, 32, 64, 128)", s.D);
  return MINITP_ERR_UNSUPPORTED;
}

int64_t decode_nsplit(int64_t S) { return cdiv(std::max<int64_t>(S, 1), CHUNK); }

}  // namespace

int64_t attention_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t S) {
  (void)T;
  (void)Hq;
  const int64_t units = B * Hkv, ns = decode_nsplit(S);
  const int64_t counters = cdiv(units * 4, 256) * 256;
  return counters + units * ns * GMAX * 2 * 4 + units * ns * GMAX * D * 4;
}

int launch_decode_attention(hipStream_t st, int dtype, const void* q, const void* k_cache, const void* v_cache,
                            void* out, const AttnShape& s, int64_t cache_len, const StepState* state, int layer,
                            void* workspace, int64_t workspace_bytes) {
  if (s.Hq % s.Hkv != 0 || s.Hq / s.Hkv > GMAX) {
    set_error("attention: Hq=%d Hkv=%d (group must divide and be <= %d)", s.Hq, s.Hkv, GMAX);
    return MINITP_ERR_UNSUPPORTED;
  }
  const int64_t need = attention_workspace_bytes(s.B, 1, s.Hq, s.Hkv, s.D, s.S);
  if (workspace_bytes < need || workspace == nullptr) {
    set_error("attention: workspace %lld B < %lld B", (long long)workspace_bytes, (long long)need);
    return MINITP_ERR_ARG;
  }
  DecodeArgs a;
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.out = out;
  a.s = s;
  a.cache_len = cache_len;
  a.st = state;
  a.layer = layer;
  a.scale = 1.0f / sqrtf((float)s.D);
  const int64_t units = (int64_t)s.B * s.Hkv;
  a.nsplit_cap = (int)decode_nsplit(s.S);
  char* ws = (char*)workspace;
  a.counters = (unsigned*)ws;
  ws += cdiv(units * 4, 256) * 256;
  a.ws_ml = (float*)ws;
  ws += units * a.nsplit_cap * GMAX * 2 * 4;
  a.ws_o = (float*)ws;
  // graph replays size the grid for a full cache; direct calls for this step
  const int64_t max_ctx = state ? s.S : cache_len + 1;
  return dtype == MINITP_F32 ? decode_by_d<float>(st, a, max_ctx) : decode_by_d<bf16>(st, a, max_ctx);
}

int launch_prefill_attention(hipStream_t st, int dtype, const void* q, const void* k_cache, const void* v_cache,
                             void* out, const AttnShape& s, int64_t cache_len) {
  if (s.Hq % s.Hkv != 0) {
    set_error("attention: Hq=%d not divisible by Hkv=%d", s.Hq, s.Hkv);
    return MINITP_ERR_ARG;
  }
  if (s.B * s.T == 0) return MINITP_OK;
  return dtype == MINITP_F32 ? prefill_by_d<float>(st, q, k_cache, v_cache, out, s, cache_len)
                             : prefill_by_d<bf16>(st, q, k_cache, v_cache, out, s, cache_len);
}

}  // namespace minitp
