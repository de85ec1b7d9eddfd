// Decode GEMV: y = epilogue(x W^T) for M <= 4 input rows, streaming W once.
//
// Layout and mapping (wave64, 256-thread blocks = 4 waves):
//  * The M input rows (optionally RMSNorm-ed, rounded to the model dtype
//    exactly as layer.py:39-42 rounds) are staged in LDS as fp32.
//  * Work unit = a "tuple" of 2P weight rows: P pairs (row_a + p, row_b + p).
//    The pairing lets an epilogue see two rows at once: SwiGLU pairs gate
//    row j with up row I + j (mlp.py:38), RoPE pairs head dims i and
//    i + D/2 (rope.py:57-62); plain stores use 2P contiguous rows.
//  * KSPLIT waves of a block share one tuple and split K; the block holds
//    4 / KSPLIT tuples and walks the tuple space with a grid stride.
//  * Each lane streams 16-byte chunks of every row of the tuple (coalesced:
//    consecutive lanes read consecutive 16 B of a row), accumulates in fp32,
//    then a butterfly reduces across the wave and LDS across the K-split.
#include "common.h"
#include "kernels.h"

namespace minitp {

namespace {

constexpr int P = 2;  // pairs per tuple (R = 4 rows)
constexpr int R = 2 * P;
constexpr int U = 2;  // chunk unroll: U * R 16-byte loads in flight per lane
constexpr int MAX_GRID = 2048;

template <int EPI>
__device__ __forceinline__ void tuple_rows(int64_t t, const GemvArgs& a, int64_t& ra, int64_t& rb) {
  if constexpr (EPI == EPI_SWIGLU) {
    ra = t * P;
    rb = a.N + t * P;
  } else if constexpr (EPI == EPI_QKV_ROPE) {
    const int half = a.a.D / 2;
    const int per_head = half / P;
    const int64_t head = t / per_head;
    ra = head * a.a.D + (t % per_head) * P;
    rb = ra + half;
  } else {
    ra = t * R;
    rb = t * R + P;
  }
}

template <int EPI>
__device__ __forceinline__ int64_t num_tuples(const GemvArgs& a) {
  if constexpr (EPI == EPI_SWIGLU) return a.N / P;
  if constexpr (EPI == EPI_QKV_ROPE) return (int64_t)(a.a.Hq + 2 * a.a.Hkv) * (a.a.D / 2) / P;
  return cdiv(a.N, R);
}

// Rows that exist in the weight matrix (contiguous tuples can overhang N).
template <int EPI>
__device__ __forceinline__ bool row_valid(int64_t r, const GemvArgs& a) {
  if constexpr (EPI == EPI_STORE || EPI == EPI_RESID || EPI == EPI_ARGMAX) return r < a.N;
  return true;
}

template <typename T, int MM, int KSPLIT, int PRO, int EPI>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  extern __shared__ float xs[];  // [MM][K]
  __shared__ float red[4][MM * R];
  __shared__ float nrm[4][MM];
  __shared__ float best_v[4][MM];
  __shared__ int64_t best_i[4][MM];
  __shared__ bool last_block;

  constexpr int V = Vec<T>::N;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t K = a.K;
  const int M = (int)a.M;
  const T* x = (const T*)a.x;

  // ---- prologue: stage (normed) input rows in LDS -------------------------
  float ss[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    ss[m] = 0.f;
    for (int64_t k = tid; k < K; k += 256) {
      float v = m < M ? load_f32<T>(x, m * a.ldx + k) : 0.f;
      xs[m * K + k] = v;
      if (PRO == PRO_NORM) ss[m] += mul_rn(v, v);
    }
  }
  if constexpr (PRO == PRO_NORM) {
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float s = wave_sum(ss[m]);
      if (lane == 0) nrm[wave][m] = s;
    }
    __syncthreads();
    const T* nw = (const T*)a.norm_w;
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float tot = (nrm[0][m] + nrm[1][m]) + (nrm[2][m] + nrm[3][m]);
      float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(tot, (float)K), a.eps)));
      for (int64_t k = tid; k < K; k += 256)
        xs[m * K + k] = m < M ? round_to<T>(mul_rn(mul_rn(xs[m * K + k], r), load_f32<T>(nw, k))) : 0.f;
    }
  }
  __syncthreads();

  // ---- main loop over tuples ------------------------------------------------
  const int kw = wave % KSPLIT;  // this wave's share of K
  const int slot = wave / KSPLIT;
  constexpr int SLOTS = 4 / KSPLIT;
  const int64_t ntup = num_tuples<EPI>(a);
  const int64_t nchunk = K / V;
  const uint4* W = (const uint4*)a.w;
  const int64_t row_chunks = nchunk;  // 16-byte chunks per weight row

  float bv[MM];
  int64_t bi[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    bv[m] = -__builtin_inff();
    bi[m] = INT64_MAX;
  }

  for (int64_t t0 = (int64_t)blockIdx.x * SLOTS; t0 < ntup; t0 += (int64_t)gridDim.x * SLOTS) {
    const int64_t t = t0 + slot;
    const bool tup_ok = t < ntup;
    int64_t ra = 0, rb = 0;
    if (tup_ok) tuple_rows<EPI>(t, a, ra, rb);
    int64_t rows[R];
    bool rok[R];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      rows[p] = ra + p;
      rows[P + p] = rb + p;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) rok[r] = tup_ok && row_valid<EPI>(rows[r], a);

    float acc[MM][R];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[m][r] = 0.f;

    for (int64_t c0 = (int64_t)kw * 64 + lane; c0 < nchunk; c0 += 64 * KSPLIT * U) {
      uint4 wv[U][R];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + (int64_t)u * 64 * KSPLIT;
#pragma unroll
        for (int r = 0; r < R; ++r)
          wv[u][r] = (rok[r] && c < nchunk) ? load_stream16(W + rows[r] * row_chunks + c)
                                            : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + (int64_t)u * 64 * KSPLIT;
        if (c < nchunk) {
          float xv[MM][V];
#pragma unroll
          for (int m = 0; m < MM; ++m)
#pragma unroll
            for (int e = 0; e < V; e += 4) {
              float4 f = *reinterpret_cast<const float4*>(&xs[m * K + c * V + e]);
              xv[m][e] = f.x;
              xv[m][e + 1] = f.y;
              xv[m][e + 2] = f.z;
              xv[m][e + 3] = f.w;
            }
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float wf[V];
            unpack16(wv[u][r], wf, (T*)nullptr);
#pragma unroll
            for (int m = 0; m < MM; ++m)
#pragma unroll
              for (int e = 0; e < V; ++e) acc[m][r] = fmaf(wf[e], xv[m][e], acc[m][r]);
          }
        }
      }
    }

    // ---- reduce: wave butterfly, then across the K-split waves in order ----
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[m][r] = wave_sum(acc[m][r]);
    if constexpr (KSPLIT > 1) {
      if (lane == 0) {
#pragma unroll
        for (int m = 0; m < MM; ++m)
#pragma unroll
          for (int r = 0; r < R; ++r) red[wave][m * R + r] = acc[m][r];
      }
      __syncthreads();
      if (kw == 0) {
#pragma unroll
        for (int m = 0; m < MM; ++m)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float s = red[wave][m * R + r];
            for (int j = 1; j < KSPLIT; ++j) s += red[wave + j][m * R + r];
            acc[m][r] = s;
          }
      }
      __syncthreads();
    }

    // ---- epilogue (waves with kw == 0; one lane per (m, pair)) -------------
    if (kw == 0 && tup_ok) {
      if constexpr (EPI == EPI_ARGMAX) {
        // every lane holds the tuple totals; fold them into the running best
        const int64_t ld = a.N;
        T* logits = (T*)a.st->logits;
#pragma unroll
        for (int m = 0; m < MM; ++m) {
          if (m < M) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
              if (rok[r]) {
                float v = round_to<T>(acc[m][r]);
                if (logits != nullptr && lane == r) store_f32<T>(logits, m * ld + rows[r], v);
                if (argmax_better(v, rows[r], bv[m], bi[m])) {
                  bv[m] = v;
                  bi[m] = rows[r];
                }
              }
            }
          }
        }
      } else {
#pragma unroll
        for (int m = 0; m < MM; ++m) {
#pragma unroll
          for (int p = 0; p < P; ++p) {
            if (lane == m * P + p && m < M) {
              float va = acc[m][p], vb = acc[m][P + p];
              const int64_t row_a = rows[p], row_b = rows[P + p];
              if constexpr (EPI == EPI_STORE) {
                T* y = (T*)a.y;
                const T* bias = (const T*)a.bias;
                if (rok[p]) store_f32<T>(y, m * a.ldy + row_a, va + (bias ? load_f32<T>(bias, row_a) : 0.f));
                if (rok[P + p]) store_f32<T>(y, m * a.ldy + row_b, vb + (bias ? load_f32<T>(bias, row_b) : 0.f));
              } else if constexpr (EPI == EPI_RESID) {
                T* y = (T*)a.y;
                const T* aux = (const T*)a.aux;
                if (rok[p])
                  store_f32<T>(y, m * a.ldy + row_a, add_rn(load_f32<T>(aux, m * a.ldy + row_a), round_to<T>(va)));
                if (rok[P + p])
                  store_f32<T>(y, m * a.ldy + row_b, add_rn(load_f32<T>(aux, m * a.ldy + row_b), round_to<T>(vb)));
              } else if constexpr (EPI == EPI_SWIGLU) {
                T* y = (T*)a.y;
                store_f32<T>(y, m * a.ldy + row_a, swiglu<T>(round_to<T>(va), round_to<T>(vb)));
              } else if constexpr (EPI == EPI_QKV_ROPE) {
                const T* bias = (const T*)a.bias;
                // F.linear output with bias, rounded to the dtype (fused.py:58)
                va = round_to<T>(va + load_f32<T>(bias, row_a));
                vb = round_to<T>(vb + load_f32<T>(bias, row_b));
                const StepState* st = a.st;
                const AttnShape& s = a.a;
                const int D = s.D, half = D / 2;
                const int64_t head = row_a / D;
                const int i = (int)(row_a % D);
                const int b = m / s.T, tt = m % s.T;
                if (head < s.Hq + s.Hkv) {
                  // rotate(x) = x * cos + rotate_half(x) * sin, fp32, each op
                  // rounded, then cast (rope.py:61-62)
                  const int64_t pos = st->positions[tt];
                  float oa, ob;
                  if (pos < 0 || pos >= a.max_pos) {
                    oa = ob = __builtin_nanf("");
                    ((StepState*)st)->error = 1;
                  } else {
                    const float* cr = a.cos_tab + pos * D;
                    const float* sr = a.sin_tab + pos * D;
                    oa = add_rn(mul_rn(va, cr[i]), -mul_rn(vb, sr[i]));
                    ob = add_rn(mul_rn(vb, cr[i + half]), mul_rn(va, sr[i + half]));
                  }
                  if (head < s.Hq) {
                    T* q = (T*)a.y;  // [B, T, Hq, D]
                    const int64_t base = ((int64_t)m * s.Hq + head) * D;
                    store_f32<T>(q, base + i, oa);
                    store_f32<T>(q, base + i + half, ob);
                  } else {
                    const int64_t g = head - s.Hq;
                    T* kc = (T*)st->k_cache + (int64_t)a.layer * s.B * s.Hkv * s.S * D;
                    const int64_t base = (((int64_t)b * s.Hkv + g) * s.S + st->cache_len + tt) * D;
                    store_f32<T>(kc, base + i, oa);
                    store_f32<T>(kc, base + i + half, ob);
                  }
                } else {
                  const int64_t g = head - s.Hq - s.Hkv;
                  T* vc = (T*)st->v_cache + (int64_t)a.layer * s.B * s.Hkv * s.S * D;
                  const int64_t base = (((int64_t)b * s.Hkv + g) * s.S + st->cache_len + tt) * D;
                  store_f32<T>(vc, base + i, va);
                  store_f32<T>(vc, base + i + half, vb);
                }
              }
            }
          }
        }
      }
    }
  }

  if constexpr (EPI == EPI_ARGMAX) {
    // block partial per row m (slots in wave order, then tuples ascending
    // inside each wave, so ties still resolve to the smallest index)
    if (kw == 0 && lane == 0) {
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        best_v[slot][m] = bv[m];
        best_i[slot][m] = bi[m];
      }
    }
    __syncthreads();
    if (tid == 0) {
      for (int m = 0; m < M; ++m) {
        float v = best_v[0][m];
        int64_t i = best_i[0][m];
        for (int s = 1; s < SLOTS; ++s)
          if (argmax_better(best_v[s][m], best_i[s][m], v, i)) {
            v = best_v[s][m];
            i = best_i[s][m];
          }
        a.part_val[(int64_t)m * gridDim.x + blockIdx.x] = v;
        a.part_idx[(int64_t)m * gridDim.x + blockIdx.x] = i;
      }
      __threadfence();
      unsigned prev = atomicAdd(a.counter, 1u);
      last_block = prev == gridDim.x - 1;
    }
    __syncthreads();
    if (last_block) {
      __threadfence();
      for (int m = 0; m < M; ++m) {
        float v = -__builtin_inff();
        int64_t i = INT64_MAX;
        for (int64_t j = tid; j < gridDim.x; j += 256) {
          float pv = __hip_atomic_load(&a.part_val[(int64_t)m * gridDim.x + j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          int64_t pi = __hip_atomic_load(&a.part_idx[(int64_t)m * gridDim.x + j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (argmax_better(pv, pi, v, i)) {
            v = pv;
            i = pi;
          }
        }
        wave_argmax(v, i);
        if (lane == 0) {
          best_v[wave][m] = v;
          best_i[wave][m] = i;
        }
      }
      __syncthreads();
      if (tid == 0) {
        for (int m = 0; m < M; ++m) {
          float v = best_v[0][m];
          int64_t i = best_i[0][m];
          for (int s = 1; s < 4; ++s)
            if (argmax_better(best_v[s][m], best_i[s][m], v, i)) {
              v = best_v[s][m];
              i = best_i[s][m];
            }
          if (a.st->next_tok != nullptr) a.st->next_tok[m * a.st->next_tok_ld] = i;
        }
        *a.counter = 0u;
      }
    }
  }
}

template <typename T, int MM, int KSPLIT, int PRO, int EPI>
int launch_cfg(hipStream_t st, const GemvArgs& a) {
  auto kern = gemv_kernel<T, MM, KSPLIT, PRO, EPI>;
  const int lds = (int)(MM * a.K * sizeof(float));
  int rc = ensure_lds_limit((const void*)kern, lds);
  if (rc) return rc;
  int64_t ntup;
  if (EPI == EPI_SWIGLU)
    ntup = a.N / P;
  else if (EPI == EPI_QKV_ROPE)
    ntup = (int64_t)(a.a.Hq + 2 * a.a.Hkv) * (a.a.D / 2) / P;
  else
    ntup = cdiv(a.N, R);
  const int64_t slots = 4 / KSPLIT;
  int grid = (int)std::min<int64_t>(cdiv(ntup, slots), EPI == EPI_ARGMAX ? gemv_argmax_partials(a.N) : MAX_GRID);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, st, a);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

template <typename T, int MM, int PRO, int EPI>
int pick_ksplit(hipStream_t st, const GemvArgs& a) {
  const int64_t nchunk = a.K / Vec<T>::N;
  if (nchunk >= 512) return launch_cfg<T, MM, 4, PRO, EPI>(st, a);
  if (nchunk >= 192) return launch_cfg<T, MM, 2, PRO, EPI>(st, a);
  return launch_cfg<T, MM, 1, PRO, EPI>(st, a);
}

template <typename T, int PRO, int EPI>
int pick_m(hipStream_t st, const GemvArgs& a) {
  if (a.M == 1) return pick_ksplit<T, 1, PRO, EPI>(st, a);
  if (a.M == 2) return pick_ksplit<T, 2, PRO, EPI>(st, a);
  return pick_ksplit<T, 4, PRO, EPI>(st, a);
}

template <typename T, int PRO>
int pick_epi(hipStream_t st, int epi, const GemvArgs& a) {
  switch (epi) {
    case EPI_STORE:
      return pick_m<T, PRO, EPI_STORE>(st, a);
    case EPI_RESID:
      return pick_m<T, PRO, EPI_RESID>(st, a);
    case EPI_SWIGLU:
      return pick_m<T, PRO, EPI_SWIGLU>(st, a);
    case EPI_QKV_ROPE:
      return pick_m<T, PRO, EPI_QKV_ROPE>(st, a);
    case EPI_ARGMAX:
      return pick_m<T, PRO, EPI_ARGMAX>(st, a);
  }
  set_error("gemv: unknown epilogue %d", epi);
  return MINITP_ERR_ARG;
}

}  // namespace

// Block count (and so partial count per row) of the LM-head argmax GEMV.
int64_t gemv_argmax_partials(int64_t N) { return std::min<int64_t>(cdiv(cdiv(N, R), 4), 1024); }

bool gemv_supported(int dtype, int64_t M, int64_t K) {
  const int64_t mm = M == 1 ? 1 : M == 2 ? 2 : 4;
  return M >= 1 && M <= 4 && mm * K * 4 <= 80 * 1024 && K % (dtype == MINITP_F32 ? 4 : 8) == 0;
}

int launch_gemv(hipStream_t st, int dtype, int pro, int epi, const GemvArgs& a) {
  if (a.M == 0 || a.N == 0) return MINITP_OK;
  if (!gemv_supported(dtype, a.M, a.K)) {
    set_error("gemv: unsupported M=%lld K=%lld", (long long)a.M, (long long)a.K);
    return MINITP_ERR_UNSUPPORTED;
  }
  if (dtype == MINITP_F32)
    return pro == PRO_NORM ? pick_epi<float, PRO_NORM>(st, epi, a) : pick_epi<float, PRO_NONE>(st, epi, a);
  return pro == PRO_NORM ? pick_epi<bf16, PRO_NORM>(st, epi, a) : pick_epi<bf16, PRO_NONE>(st, epi, a);
}

}  // namespace minitp
