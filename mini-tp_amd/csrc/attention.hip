// GQA attention over the KV cache (attention.py:77-105 at tp_size == 1).
//
// Q head h reads KV head h / G (G = Hq / Hkv), the order repeat_interleave
// gives (attention.py:89-90), so no K/V copy is ever made. Scale 1/sqrt(D)
// (SDPA default). Softmax and accumulation in fp32; the output is rounded to
// the model dtype once.
#include <cstddef>

#include "common.h"
#include "kernels.h"

namespace minitp {

namespace {

constexpr int GMAX = 8;  // max q heads per KV head served
constexpr int NW = 8;    // waves per decode block

__device__ __forceinline__ uint4 attn_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Decode geometry: a lane owns 8 consecutive elements of a key row, so LPR
// lanes cover a row and one load instruction of a wave covers PPI rows. A
// wave chunk is NI such loads (CP key positions).
template <int D>
struct DecodeGeom {
  static constexpr int LPR = D / 8;
  static constexpr int PPI = 64 / LPR;
  static constexpr int NI = LPR < 8 ? LPR : 8;
  static constexpr int CP = NI * PPI;
  static constexpr int DUP = LPR / NI;  // lanes holding the same reduced score
};

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
  float* ws_ml;  // [B * Hkv][nsplit][GMAX][2]  (split partials, nsplit > 1)
  float* ws_o;   // [B * Hkv][nsplit][GMAX][D]
  // Arrival words, one per (batch row, KV head), zero between launches
  // (the forward's step state holds them): when set, the MFMA kernel's last
  // split block of a unit merges the splits itself (no merge launch).
  uint32_t* count;
  OprojArgs op;  // decode_attn_kernel<..., NLW > 0>: the folded o_proj
};

// The caches and cache_len of a decode launch: from the step state inside a
// forward (one branch, the three fields loaded together rather than one
// dependent scalar load per use), else the launch's own values.
struct DecodeKV {
  const void* k;
  const void* v;
  int64_t cache_len;
};
__device__ __forceinline__ DecodeKV decode_kv(const DecodeArgs& a, int64_t layer_off, int64_t elem_bytes) {
  DecodeKV r{a.k, a.v, a.cache_len};
  if (a.st != nullptr) {
    const StepArgs& sa = a.st->args;
    r.cache_len = sa.cache_len;
    r.k = (const char*)sa.k_cache + layer_off * elem_bytes;
    r.v = (const char*)sa.v_cache + layer_off * elem_bytes;
  }
  return r;
}

// 16-byte load of streamed weights (read once per step: non-temporal).
__device__ __forceinline__ uint4 weight_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Value held by lane j ^ (2 * MK - 1) (rows of 16 lanes, DPP). Used for a
// reduce-scatter whose masks fall from high to low: the bits above MK are
// already equal between the two lanes and the bits below are still free.
template <int MK>
__device__ __forceinline__ float flip_low(float v) {
  static_assert(MK == 1 || MK == 2 || MK == 4 || MK == 8, "mask within a row");
  if constexpr (MK == 1) return dpp_f32<0xB1>(0.f, v);   // quad_perm [1,0,3,2]
  if constexpr (MK == 2) return dpp_f32<0x1B>(0.f, v);   // quad_perm [3,2,1,0]
  if constexpr (MK == 4) return dpp_f32<0x141>(0.f, v);  // row_half_mirror
  if constexpr (MK == 8) return dpp_f32<0x140>(0.f, v);  // row_mirror
}

// Scores: v[r][h] holds this lane's partial dot for load r, head h. Sum over
// the LPR lanes of a row, scattering r: afterwards v[0][h] is the full score
// of load (lane % LPR) / DUP.
template <int N, int MK, int GP>
__device__ __forceinline__ void score_scatter(float (&v)[8][GP], int lane) {
  if constexpr (MK >= 1) {
    if constexpr (N > 1) {
      const bool hi = lane & MK;
#pragma unroll
      for (int r = 0; r < N / 2; ++r)
#pragma unroll
        for (int h = 0; h < GP; ++h) {
          const float keep = hi ? v[r + N / 2][h] : v[r][h];
          const float send = hi ? v[r][h] : v[r + N / 2][h];
          v[r][h] = keep + flip_low<MK>(send);
        }
      score_scatter<N / 2, MK / 2, GP>(v, lane);
    } else {
#pragma unroll
      for (int h = 0; h < GP; ++h) v[0][h] += flip_low<MK>(v[0][h]);
      score_scatter<1, MK / 2, GP>(v, lane);
    }
  }
}

// Output: a[h * 8 + e] is this lane's partial for head h, element e of its
// slice. Sum over the lanes sharing the slice (lane masks MK, 2 MK, ... 32);
// the first steps scatter the flat index, later ones (once one value is
// left) are plain sums.
template <int N, int MK, int NA>
__device__ __forceinline__ void out_scatter(float (&a)[NA], int lane) {
  if constexpr (MK < 64) {
    if constexpr (N > 1) {
      const bool hi = lane & MK;
#pragma unroll
      for (int i = 0; i < N / 2; ++i) {
        const float keep = hi ? a[i + N / 2] : a[i];
        const float send = hi ? a[i] : a[i + N / 2];
        a[i] = keep + __shfl_xor(send, MK, 64);
      }
      out_scatter<N / 2, MK * 2, NA>(a, lane);
    } else {
      a[0] += __shfl_xor(a[0], MK, 64);
      out_scatter<1, MK * 2, NA>(a, lane);
    }
  }
}

template <typename T>
__device__ __forceinline__ float dot8(const uint4 (&k)[sizeof(T) / 2], const T* q) {
  if constexpr (sizeof(T) == 2) {
    const uint4 qv = *reinterpret_cast<const uint4*>(q);
    float acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k[0].x),
                                                __builtin_bit_cast(bf16x2_t, qv.x), 0.f, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k[0].y), __builtin_bit_cast(bf16x2_t, qv.y),
                                          acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k[0].z), __builtin_bit_cast(bf16x2_t, qv.z),
                                          acc, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k[0].w), __builtin_bit_cast(bf16x2_t, qv.w),
                                           acc, false);
  } else {
    const float4 q0 = *reinterpret_cast<const float4*>(q);
    const float4 q1 = *reinterpret_cast<const float4*>(q + 4);
    float acc = __uint_as_float(k[0].x) * q0.x;
    acc = fmaf(__uint_as_float(k[0].y), q0.y, acc);
    acc = fmaf(__uint_as_float(k[0].z), q0.z, acc);
    acc = fmaf(__uint_as_float(k[0].w), q0.w, acc);
    acc = fmaf(__uint_as_float(k[1].x), q1.x, acc);
    acc = fmaf(__uint_as_float(k[1].y), q1.y, acc);
    acc = fmaf(__uint_as_float(k[1].z), q1.z, acc);
    return fmaf(__uint_as_float(k[1].w), q1.w, acc);
  }
}

template <typename T>
__device__ __forceinline__ void unpack8(const uint4 (&v)[sizeof(T) / 2], float (&f)[8]) {
  if constexpr (sizeof(T) == 2) {
    unpack16(v[0], f, (bf16*)nullptr);
  } else {
    unpack16(v[0], f, (float*)nullptr);
    unpack16(v[1], f + 4, (float*)nullptr);
  }
}

// Orders LDS traffic between the lanes of one wave (no hardware barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One block per (batch row, KV head, split, group of HP query heads). Its NW
// waves take CP-position chunks of the cache in turn (chunk c goes to split
// c % nsplit); each wave keeps an online softmax for its HP heads, so a wave
// never waits on another until the end, where the waves merge through LDS.
// Inside a chunk a lane loads 8 elements of NI key rows and of NI value rows
// in one go (16-byte loads, a row spread over LPR lanes), reduces the scores
// over the row's lanes with DPP, and reads the probabilities of the rows it
// holds back from wave-private LDS for P V. A wave's VALU work per chunk
// grows with HP: small batches run HP = 1 (more blocks, K/V re-read from
// L2 per head), large ones the whole group (K/V read once).
//
// NLW > 0 folds o_proj in (one batch row, HP = 1, one split; gridDim.y is
// the number of W_o row slices): every block loads its slice of W_o (rows
// blockIdx.y * rows .., the D columns of its head; NLW 16-byte loads per
// thread) before the attention, rounds the head's output to the dtype (the
// SDPA output, attention.py:92-105) and writes o . W_o[row, head columns] as
// fp32 partial rows part[head][row]. Each row's D-element dot is one chunk
// per lane (a fixed fmaf chain) plus a butterfly over the row's lanes.
template <typename T, int D, int HP, int NLW = 0>
__global__ __launch_bounds__(NW * 64) void decode_attn_kernel(DecodeArgs a) {
  using Geo = DecodeGeom<D>;
  constexpr int LPR = Geo::LPR, PPI = Geo::PPI, NI = Geo::NI, CP = Geo::CP, DUP = Geo::DUP;
  constexpr int U = (int)sizeof(T) / 2;  // 16-byte loads per 8 elements
  constexpr int NA = HP * 8;             // output partials per lane
  __shared__ __attribute__((aligned(16))) T qs[HP][D];
  __shared__ __attribute__((aligned(16))) float ps[NW][CP][HP];
  __shared__ __attribute__((aligned(16))) float po[NW][HP][D];
  __shared__ float pm[NW][HP], pl[NW][HP];

  const AttnShape& s = a.s;
  const int G = s.Hq / s.Hkv;
  const int bh = blockIdx.x, b = bh / s.Hkv, g = bh % s.Hkv;
  const int split = NLW > 0 ? 0 : (int)blockIdx.y, nsplit = NLW > 0 ? 1 : (int)gridDim.y;
  const int h0 = blockIdx.z * HP;  // first query head (within the group) of this block
  const int nh = std::min(HP, G - h0);
  const int64_t layer_off = (int64_t)a.layer * s.B * s.Hkv * s.S * D;
  const DecodeKV kv = decode_kv(a, layer_off, (int64_t)sizeof(T));
  const int64_t ctx = kv.cache_len + 1;
  const int64_t nchunk = cdiv(ctx, CP);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int col = lane % LPR, grow = lane / LPR;
  const int rbase = col / DUP;
  const bool owner = col % DUP == 0;

  const T* kc = (const T*)kv.k + (int64_t)bh * s.S * D;
  const T* vc = (const T*)kv.v + (int64_t)bh * s.S * D;

  // The context's K / V rows through resources that end at row ctx (rows past
  // it read zeros, so the loads are unconditional), and this wave's first
  // chunk requested before the query: its addresses do not depend on the
  // query, so the two memory round trips overlap.
  const uint32_t kv_bytes = (uint32_t)(ctx * D * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t krs = span_rsrc(kc, kv_bytes), vrs = span_rsrc(vc, kv_bytes);
  uint4 kr[NI][U], vr[NI][U];
  auto load_chunk = [&](int64_t c) {
#pragma unroll
    for (int r = 0; r < NI; ++r) {
      const uint32_t off = (uint32_t)(((c * CP + r * PPI + grow) * D + col * 8) * (int64_t)sizeof(T));
#pragma unroll
      for (int u = 0; u < U; ++u) {
        kr[r][u] = attn_load16(krs, off + 16 * u);
        vr[r][u] = attn_load16(vrs, off + 16 * u);
      }
    }
  };
  const int64_t c_first = (int64_t)w * nsplit + split;
  load_chunk(c_first);

  {
    const T* q = (const T*)a.q + ((int64_t)b * s.Hq + (int64_t)g * G + h0) * D;
    for (int i = tid; i < HP * D; i += NW * 64) (&qs[0][0])[i] = i < nh * D ? q[i] : T{};
  }
  __syncthreads();

  // (NLW > 0) this block's W_o slice, in flight during the attention
  constexpr int OV = Vec<T>::N, CPR = D / OV;  // elements per load; loads per row segment
  static_assert(NLW == 0 || (HP == 1 && CPR >= 1 && CPR <= 64 && (64 % CPR) == 0), "o_proj slice layout");
  uint4 wo[NLW > 0 ? NLW : 1];
  int64_t orow0 = 0, onrows = 0;
  if constexpr (NLW > 0) {
    const int hq = g * G + h0;
    orow0 = (int64_t)blockIdx.y * a.op.rows;
    onrows = std::min<int64_t>(a.op.rows, a.op.H - orow0);
    const int64_t ldw = (int64_t)s.Hq * D;
    const __amdgpu_buffer_rsrc_t wr =
        span_rsrc((const T*)a.op.w + orow0 * ldw + (int64_t)hq * D, (uint32_t)(onrows * ldw * sizeof(T)));
#pragma unroll
    for (int i = 0; i < NLW; ++i) {
      const int f = tid + i * NW * 64;
      wo[i] = weight_load16(wr, (uint32_t)(((int64_t)(f / CPR) * ldw + (f % CPR) * OV) * sizeof(T)));
    }
  }

  float m[HP], lsum[HP], acc[NA];
#pragma unroll
  for (int h = 0; h < HP; ++h) {
    m[h] = -__builtin_inff();
    lsum[h] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < NA; ++i) acc[i] = 0.f;

  for (int64_t c = c_first; c < nchunk; c += (int64_t)NW * nsplit) {
    const int64_t p0 = c * CP;
    if (c != c_first) load_chunk(c);
    // scores of this lane's 8-element slices, summed across each row
    float sc[8][HP];
#pragma unroll
    for (int r = 0; r < NI; ++r)
#pragma unroll
      for (int h = 0; h < HP; ++h) sc[r][h] = dot8<T>(kr[r], &qs[h][col * 8]);
    score_scatter<NI, LPR / 2, HP>(sc, lane);
    const int prow = rbase * PPI + grow;  // chunk row whose score this lane holds
    const bool valid = p0 + prow < ctx;
    float alpha[HP];
#pragma unroll
    for (int h = 0; h < HP; ++h) {
      const float sv = valid ? sc[0][h] * a.scale : -__builtin_inff();
      const float mn = fmaxf(m[h], wave_max(sv));  // finite: the chunk's first row is valid
      alpha[h] = expf(m[h] - mn);
      const float p = expf(sv - mn);
      sc[0][h] = p;
      lsum[h] = fmaf(lsum[h], alpha[h], owner ? p : 0.f);
      m[h] = mn;
    }
    if (owner) {
#pragma unroll
      for (int h = 0; h < HP; ++h) ps[w][prow][h] = sc[0][h];
    }
    wave_lds_sync();
#pragma unroll
    for (int h = 0; h < HP; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h * 8 + e] *= alpha[h];
#pragma unroll
    for (int r = 0; r < NI; ++r) {
      float vf[8], pr[HP];
      unpack8<T>(vr[r], vf);
#pragma unroll
      for (int h = 0; h < HP; ++h) pr[h] = ps[w][r * PPI + grow][h];
#pragma unroll
      for (int h = 0; h < HP; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h * 8 + e] = fmaf(pr[h], vf[e], acc[h * 8 + e]);
    }
    wave_lds_sync();
  }

  // ---- wave results -> LDS ---------------------------------------------------
  out_scatter<NA, LPR, NA>(acc, lane);
  {
    // flat indices [ibase, ibase + nv) survive in this lane
    constexpr int STEPS = __builtin_ctz(PPI);
    constexpr int SC = __builtin_ctz(NA) < STEPS ? __builtin_ctz(NA) : STEPS;
    constexpr int NV = NA >> SC;
    int ibase = 0;
#pragma unroll
    for (int j = 0; j < SC; ++j) ibase += ((grow >> j) & 1) * (NA >> (j + 1));
    const bool out_owner = (grow >> SC) == 0;
    if (out_owner) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int f = ibase + i, h = f / 8, e = f % 8;
        po[w][h][col * 8 + e] = acc[i];
      }
    }
  }
#pragma unroll
  for (int h = 0; h < HP; ++h) {
    const float l = wave_sum(lsum[h]);
    if (lane == 0) {
      pm[w][h] = m[h];
      pl[w][h] = l;
    }
  }
  __syncthreads();

  // ---- merge the waves ---------------------------------------------------------
  T* out = (T*)a.out;
  for (int i = tid; i < nh * D; i += NW * 64) {
    const int h = i / D, d = i % D;
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < NW; ++j) mx = fmaxf(mx, pm[j][h]);
    float l = 0.f, o = 0.f;
    if (mx != -__builtin_inff()) {
#pragma unroll
      for (int j = 0; j < NW; ++j) {
        if (pm[j][h] == -__builtin_inff()) continue;  // wave saw no chunk
        const float sc = expf(pm[j][h] - mx);
        l = fmaf(sc, pl[j][h], l);
        o = fmaf(sc, po[j][h][d], o);
      }
    }
    if constexpr (NLW > 0) {
      po[0][0][d] = round_to<T>(o / l);  // (element d is read and written by this thread only)
    } else if (nsplit == 1) {
      store_f32<T>(out, ((int64_t)b * s.Hq + g * G + h0 + h) * D + d, o / l);
    } else {
      const int64_t slot = ((int64_t)bh * nsplit + split) * GMAX + h0 + h;
      a.ws_o[slot * D + d] = o;
      if (d == 0) {
        a.ws_ml[slot * 2] = mx;
        a.ws_ml[slot * 2 + 1] = l;
      }
    }
  }

  // ---- (NLW > 0) o_proj partial of this head over the block's rows -------------
  if constexpr (NLW > 0) {
    __syncthreads();
    float* part = a.op.part + (int64_t)(g * G + h0) * a.op.H + orow0;
#pragma unroll
    for (int i = 0; i < NLW; ++i) {
      const int f = tid + i * NW * 64, row = f / CPR, c = f % CPR;
      float wf[OV];
      unpack16(wo[i], wf, (T*)nullptr);
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < OV; ++e) acc = fmaf(wf[e], po[0][0][c * OV + e], acc);
#pragma unroll
      for (int o = CPR / 2; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
      if (c == 0 && row < onrows) part[row] = acc;
    }
  }
}

// Merge of the splits of each (batch row, KV head) (a separate launch, so
// the partials are visible without any grid-wide fence). Block (bh, part)
// takes MERGE_T of the group's G x D outputs; a thread loads the partials
// of MERGE_NS splits at once (one memory round trip for nsplit <= MERGE_NS)
// and folds them into a running (max, sum, output) in split order.
constexpr int MERGE_T = 128;
constexpr int MERGE_NS = 8;

// Output (h, d) of unit bh from its nsplit partials. DEV: the partials were
// stored by other blocks of the same launch (device-coherent loads).
template <bool DEV>
__device__ __forceinline__ float ws_load(const float* p) {
  if constexpr (DEV) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return *p;
}
template <int D, bool DEV>
__device__ __forceinline__ float merge_splits(const DecodeArgs& a, int bh, int nsplit, int h, int d) {
  float mx = -__builtin_inff(), l = 0.f, o = 0.f;
  for (int sp0 = 0; sp0 < nsplit; sp0 += MERGE_NS) {
    float ms[MERGE_NS], ls[MERGE_NS], os[MERGE_NS];
#pragma unroll
    for (int u = 0; u < MERGE_NS; ++u) {
      const int sp = sp0 + u < nsplit ? sp0 + u : sp0;
      const int64_t slot = ((int64_t)bh * nsplit + sp) * GMAX + h;
      ms[u] = sp0 + u < nsplit ? ws_load<DEV>(a.ws_ml + slot * 2) : -__builtin_inff();
      ls[u] = ws_load<DEV>(a.ws_ml + slot * 2 + 1);
      os[u] = ws_load<DEV>(a.ws_o + slot * D + d);
    }
    float cm = mx;
#pragma unroll
    for (int u = 0; u < MERGE_NS; ++u) cm = fmaxf(cm, ms[u]);
    if (cm == -__builtin_inff()) continue;  // no split of this chunk saw a position yet
    const float alpha = mx == -__builtin_inff() ? 0.f : expf(mx - cm);
    l *= alpha;
    o *= alpha;
#pragma unroll
    for (int u = 0; u < MERGE_NS; ++u) {
      if (ms[u] == -__builtin_inff()) continue;  // split saw no position
      const float sc = expf(ms[u] - cm);
      l = fmaf(sc, ls[u], l);
      o = fmaf(sc, os[u], o);
    }
    mx = cm;
  }
  return o / l;
}

template <typename T, int D>
__global__ __launch_bounds__(MERGE_T) void decode_merge_kernel(DecodeArgs a, int nsplit) {
  const AttnShape& s = a.s;
  const int G = s.Hq / s.Hkv;
  const int bh = blockIdx.x, b = bh / s.Hkv, g = bh % s.Hkv;
  const int i = blockIdx.y * MERGE_T + threadIdx.x;
  if (i >= G * D) return;
  const int h = i / D, d = i % D;
  store_f32<T>((T*)a.out, ((int64_t)b * s.Hq + g * G + h) * D + d, merge_splits<D, false>(a, bh, nsplit, h, d));
}

// ---------------------------------------------------------------------------
// Grouped decode attention on MFMA (bf16, D = 64 or 128, G <= GMAX query
// heads per KV head). The G heads of a KV group are the 16-row side of
// v_mfma_f32_16x16x32_bf16 (rows G..15 zero): the scores of 16 key positions
// are D / 32 MFMAs (A: lane l holds q head l % 16, dims 32 s + 8 (l / 16)
// .. +7; B: key row p + l % 16, the same dims) and P V of 32 positions is
// D / 16 MFMAs. P V wants each lane's 8 consecutive positions of one V
// column and of one P row, so both pass through wave-private LDS: the V tile
// row-major with a row stride of 2 D + 8 bytes (the four lane groups' 16-bit
// column reads, 8 rows apart, land in different banks), P as [head][position]
// bf16 rows of 80 bytes (one conflict-free 16-byte read per lane). Softmax
// per head in fp32 (base 2, the 1/sqrt(D) scale folded into the exponent);
// P is rounded to bf16 for its MFMA.
// Block = NWM waves over one split's position range, 32-position tiles
// round robin, each tile's K and V loads issued before the previous tile's
// math. Waves merge in LDS; splits merge as in decode_attn_kernel (same
// workspace layout and merge arithmetic), inside a forward by the unit's
// last split block (arrival words in the step state), else by the merge
// kernel. Measured at batch 32 (0.5B shape, context about 2,300): 4 splits
// of 8 waves 13.3 us a layer with the in-kernel merge (10.5 + 4.8 us with
// the merge kernel); 1, 2, 6 or 8 splits, 16 waves, or three tiles of
// loads in flight per wave were all slower or no faster.
#ifndef MINITP_DEC_MF_WAVES
#define MINITP_DEC_MF_WAVES 8
#endif
constexpr int NWM = MINITP_DEC_MF_WAVES;
typedef __bf16 bf16x8_a __attribute__((ext_vector_type(8)));
typedef float f32x4_a __attribute__((ext_vector_type(4)));

template <int D>
struct MfDec {
  static constexpr int VS = 2 * D + 8;         // V tile row stride in LDS (bytes)
  static constexpr int PS = 80;                // P row stride in LDS (bytes)
  static constexpr int VL = D / 16;            // 16-byte V loads per lane per tile (32 rows x D)
  static constexpr int WAVE_LDS = 32 * VS + 16 * PS;
};

template <int D>
__global__ __launch_bounds__(NWM * 64) void decode_attn_mfma_kernel(DecodeArgs a) {
  using Geo = MfDec<D>;
  constexpr int KS = D / 32;   // 32-dim steps of the scores
  constexpr int DB = D / 16;   // 16-column blocks of the output
  constexpr int VL = Geo::VL;
  constexpr uint32_t OOB = 0xffffffffu;
  extern __shared__ __attribute__((aligned(16))) char lds[];  // NWM * Geo::WAVE_LDS
  __shared__ float pm[NWM][GMAX], pl[NWM][GMAX];

  const AttnShape& s = a.s;
  const int G = s.Hq / s.Hkv;
  const int bh = blockIdx.x, b = bh / s.Hkv, g = bh % s.Hkv;
  const int split = blockIdx.y, nsplit = gridDim.y;
  const int64_t layer_off = (int64_t)a.layer * s.B * s.Hkv * s.S * D;
  const DecodeKV kv = decode_kv(a, layer_off, 2);
  const int64_t ctx = kv.cache_len + 1;
  // the wave index made explicitly uniform: the tile loop then runs on scalar
  // branches, and the compiler counts the loads in flight across it exactly
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, q4 = lane >> 4;
  char* vs = lds + w * Geo::WAVE_LDS;
  char* ps = vs + 32 * Geo::VS;

  const int64_t tiles = cdiv(ctx, (int64_t)32);
  const int64_t span = cdiv(tiles, (int64_t)nsplit);
  const int64_t t_begin = split * span, t_end = std::min(tiles, t_begin + span);

  const bf16* kc = (const bf16*)kv.k + (int64_t)bh * s.S * D;
  const bf16* vc = (const bf16*)kv.v + (int64_t)bh * s.S * D;
  const uint32_t kv_bytes = (uint32_t)(ctx * D * 2);  // rows past the context read zeros
  const __amdgpu_buffer_rsrc_t kr = span_rsrc(kc, kv_bytes), vr = span_rsrc(vc, kv_bytes);

  // q heads of the group as the A operand (rows G..15 zero)
  bf16x8_a qa[KS];
  {
    const bf16* qp = (const bf16*)a.q + ((int64_t)b * s.Hq + (int64_t)g * G) * D;
    const __amdgpu_buffer_rsrc_t qr = span_rsrc(qp, (uint32_t)(G * D * 2));
#pragma unroll
    for (int k = 0; k < KS; ++k)
      qa[k] = __builtin_bit_cast(bf16x8_a, attn_load16(qr, n16 < G ? (uint32_t)((n16 * D + 32 * k + 8 * q4) * 2) : OOB));
  }

  // loads of one tile: K as B operands (two 16-position halves x KS steps),
  // V rows for the LDS stage (lane l: row l % 32, dims (l / 32) D / 2 ..)
  struct Tile {
    uint4 k[2][KS];
    uint4 v[VL];
  };
  auto issue = [&](Tile& tl, int64_t t) {
    const bool live = t < t_end;
    const int64_t p0 = t * 32;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int k = 0; k < KS; ++k)
        tl.k[h][k] = attn_load16(kr, live ? (uint32_t)(((p0 + 16 * h + n16) * D + 32 * k + 8 * q4) * 2) : OOB);
#pragma unroll
    for (int i = 0; i < VL; ++i)
      tl.v[i] = attn_load16(vr, live ? (uint32_t)(((p0 + (lane & 31)) * D + (lane >> 5) * (D / 2) + 8 * i) * 2) : OOB);
  };

  const float sl2 = a.scale * 1.4426950408889634f;  // scores to base-2 exponent units
  float m[4], l[4];
  f32x4_a o[DB];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m[r] = -__builtin_inff();
    l[r] = 0.f;
  }
#pragma unroll
  for (int c = 0; c < DB; ++c) o[c] = f32x4_a{0.f, 0.f, 0.f, 0.f};

  Tile cur, nxt;
  int64_t t = t_begin + w;
  issue(cur, t);
  for (; t < t_end; t += NWM) {
    issue(nxt, t + NWM);
    // V tile -> LDS, row-major (two 8-byte writes per 16-byte piece)
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      char* dst = vs + (lane & 31) * Geo::VS + ((lane >> 5) * (D / 2) + 8 * i) * 2;
      *(uint2*)dst = make_uint2(cur.v[i].x, cur.v[i].y);
      *(uint2*)(dst + 8) = make_uint2(cur.v[i].z, cur.v[i].w);
    }
    // scores: lane l holds head 4 (l / 16) + r, position p0 + 16 h + l % 16
    f32x4_a sc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sc[h] = f32x4_a{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < KS; ++k)
        sc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[k], __builtin_bit_cast(bf16x8_a, cur.k[h][k]), sc[h], 0, 0, 0);
    }
    const int64_t p0 = t * 32;
    float pv[2][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float x0 = p0 + n16 < ctx ? sc[0][r] * sl2 : -__builtin_inff();
      float x1 = p0 + 16 + n16 < ctx ? sc[1][r] * sl2 : -__builtin_inff();
      float mx = fmaxf(x0, x1);
      mx = fmaxf(mx, flip_low<1>(mx));
      mx = fmaxf(mx, flip_low<2>(mx));
      mx = fmaxf(mx, flip_low<4>(mx));
      mx = fmaxf(mx, flip_low<8>(mx));
      const float mn = fmaxf(m[r], mx);  // finite: the tile's first position is valid
      const float alpha = __builtin_amdgcn_exp2f(m[r] - mn);
      const float e0 = __builtin_amdgcn_exp2f(x0 - mn), e1 = __builtin_amdgcn_exp2f(x1 - mn);
      float sum = e0 + e1;
      sum += flip_low<1>(sum);
      sum += flip_low<2>(sum);
      sum += flip_low<4>(sum);
      sum += flip_low<8>(sum);
      l[r] = fmaf(l[r], alpha, sum);
      m[r] = mn;
#pragma unroll
      for (int c = 0; c < DB; ++c) o[c][r] *= alpha;
      pv[0][r] = e0;
      pv[1][r] = e1;
    }
    // P -> LDS as [head][position] bf16
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *(uint16_t*)(ps + (4 * q4 + r) * Geo::PS + (16 * h + n16) * 2) = f32_to_bf16(pv[h][r]);
    wave_lds_sync();
    // P V: A = P (head l % 16, positions 8 (l / 16) .. +7), B = V column
    // block c (positions 8 (l / 16) .. +7 of column 16 c + l % 16)
    const bf16x8_a pa = __builtin_bit_cast(bf16x8_a, *(const uint4*)(ps + n16 * Geo::PS + 16 * q4));
#pragma unroll
    for (int c = 0; c < DB; ++c) {
      uint32_t vw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const char* src = vs + (8 * q4 + 2 * e) * Geo::VS + (16 * c + n16) * 2;
        vw[e] = (uint32_t)*(const uint16_t*)src | ((uint32_t)*(const uint16_t*)(src + Geo::VS) << 16);
      }
      o[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, __builtin_bit_cast(bf16x8_a, make_uint4(vw[0], vw[1], vw[2], vw[3])),
                                                    o[c], 0, 0, 0);
    }
    wave_lds_sync();  // this tile's LDS reads done before the next tile's writes
    cur = nxt;
  }

  // ---- the waves' states -> LDS (the V stage is free now) -------------------
  float* po = (float*)vs;  // [GMAX][D] of this wave
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * q4 + r;
    if (h < G) {
#pragma unroll
      for (int c = 0; c < DB; ++c) po[h * D + 16 * c + n16] = o[c][r];
      if (n16 == 0) {
        pm[w][h] = m[r];
        pl[w][h] = l[r];
      }
    }
  }
  __syncthreads();

  // ---- merge the waves (m in base-2 units) ---------------------------------
  bf16* out = (bf16*)a.out;
  for (int i = tid; i < G * D; i += NWM * 64) {
    const int h = i / D, d = i % D;
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < NWM; ++j) mx = fmaxf(mx, pm[j][h]);
    float lsum = 0.f, acc = 0.f;
    if (mx != -__builtin_inff()) {
#pragma unroll
      for (int j = 0; j < NWM; ++j) {
        if (pm[j][h] == -__builtin_inff()) continue;  // wave saw no tile
        const float sc = __builtin_amdgcn_exp2f(pm[j][h] - mx);
        lsum = fmaf(sc, pl[j][h], lsum);
        acc = fmaf(sc, ((const float*)(lds + j * Geo::WAVE_LDS))[h * D + d], acc);
      }
    }
    if (nsplit == 1) {
      store_f32<bf16>(out, ((int64_t)b * s.Hq + g * G + h) * D + d, acc / lsum);
    } else {
      // the merge works in natural-log units
      const int64_t slot = ((int64_t)bh * nsplit + split) * GMAX + h;
      const float mln = mx == -__builtin_inff() ? mx : mx * 0.6931471805599453f;
      if (a.count != nullptr) {  // device-coherent (sc1): read by the unit's last block
        __hip_atomic_store(a.ws_o + slot * D + d, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == 0) {
          __hip_atomic_store(a.ws_ml + slot * 2, mln, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(a.ws_ml + slot * 2 + 1, lsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else {
        a.ws_o[slot * D + d] = acc;
        if (d == 0) {
          a.ws_ml[slot * 2] = mln;
          a.ws_ml[slot * 2 + 1] = lsum;
        }
      }
    }
  }
  if (nsplit == 1 || a.count == nullptr) return;

  // ---- in-kernel merge: the unit's last split block to arrive -------------
  // Every wave's partial stores complete (vmcnt(0) expcnt(7) lgkmcnt(15))
  // before the block is counted in: an agent-scope release without its
  // whole-L2 write-back. The last block merges in split order (the same
  // result whatever the arrival order) and puts the word back to 0.
  __shared__ int last_blk;
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(a.count + bh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_blk = old == (uint32_t)(nsplit - 1);
    if (last_blk) __hip_atomic_store(a.count + bh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last_blk) return;
  for (int i = tid; i < G * D; i += NWM * 64) {
    const int h = i / D, d = i % D;
    store_f32<bf16>(out, ((int64_t)b * s.Hq + g * G + h) * D + d, merge_splits<D, true>(a, bh, nsplit, h, d));
  }
}

// Inside a forward (st != null) a prompt's attention takes the layer's
// caches and cache_len from the step state, as the decode kernels do, so a
// captured prompt graph replays for other caches and positions; direct calls
// pass them by value.
struct PrefillKV {
  const StepState* st;
  int64_t layer_off;  // elements from a cache base to this layer's [B, Hkv, S, D]
  template <typename T>
  __device__ __forceinline__ void resolve(const T*& kc, const T*& vc, int64_t& cache_len) const {
    if (st != nullptr) {
      kc = (const T*)st->args.k_cache + layer_off;
      vc = (const T*)st->args.v_cache + layer_off;
      cache_len = st->args.cache_len;
    }
  }
};

// ---------------------------------------------------------------------------
// Prefill: flash-style causal attention, fp32 FMA. Block = (b * Hq + h,
// 64-query tile); 4 lanes per query, each owning D/4 dims; key tiles of K
// and V (64 keys, 32 at D = 128) staged in LDS as fp32.
constexpr int QT = 64;

template <typename T, int D>
__global__ __launch_bounds__(256) void prefill_attn_kernel(const T* q, const T* kc, const T* vc, T* out, AttnShape s,
                                                           int64_t cache_len, float scale, PrefillKV kv) {
  kv.resolve(kc, vc, cache_len);
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


// Prefill on matrix cores (bf16): block = (b * Hq + h, PQ-query tile), wave
// w = the 16-query strip t0 = PQ y + 16 w (all strips share each staged tile). Per 64-key tile staged in LDS (K
// row-major, V transposed so that a V operand is 4 consecutive keys), the
// products run transposed: S^T = K Q^T by MFMA 16x16x16 leaves lane
// (q, r) holding keys 4q .. 4q + 3 of query r, which is exactly its B operand
// of O^T = V^T P^T, so the probabilities (rounded to bf16) never leave the
// registers and each lane's softmax state (max, sum; base 2) and O^T column
// belong to its own query: a tile's max needs two xor shuffles and the
// rescale none. The row sums stay per lane in fp32 and are added across the
// four lanes of a query at the end; O / l is rounded to bf16 once.
// PW waves (16-query strips) per block, PQ = 16 PW queries.
template <int D, int PW>
__global__ __launch_bounds__(PW * 64) void prefill_attn_mfma_kernel(const bf16* q, const bf16* kc, const bf16* vc,
                                                                    bf16* out, AttnShape s, int64_t cache_len,
                                                                    float scale, PrefillKV kv) {
  kv.resolve(kc, vc, cache_len);
  constexpr int PQ = 16 * PW;
  typedef short short4_t __attribute__((ext_vector_type(4)));
  typedef float float4_t __attribute__((ext_vector_type(4)));
  constexpr int KT = 64;            // keys per tile
  constexpr int KB = KT / 16;       // 16-key blocks per tile
  constexpr int KS = D / 16;        // 16-dim steps of a score, and 16-dim output blocks
  constexpr int PPRW = D / 8;       // 16-byte pieces per K / V row
  constexpr int KROW = D * 2 + 16;  // LDS bytes per K row (padded)
  constexpr int VROW = KT * 2 + 8;  // LDS bytes per transposed V row (one dim)
  __shared__ __attribute__((aligned(16))) char Ks[KT * KROW];
  __shared__ __attribute__((aligned(16))) char Vt[D * VROW];
  const int G = s.Hq / s.Hkv;
  const int bh = blockIdx.x, b = bh / s.Hq, h = bh % s.Hq, g = h / G;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane % 16, lq = lane / 16;
  const int64_t t0 = (int64_t)blockIdx.y * PQ + wave * 16;
  const bf16* kbase = kc + ((int64_t)b * s.Hkv + g) * s.S * D;
  const bf16* vbase = vc + ((int64_t)b * s.Hkv + g) * s.S * D;
  const float sl2 = scale * 1.4426950408889634f;

  // head dims that are a multiple of 32 run gfx950's 16x16x32 MFMA (8 bf16 per
  // lane per operand: k = 8 (lane / 16) + e), 16 keeps 16x16x16 (k = 4 (lane / 16) + e)
  constexpr bool W32 = D % 32 == 0;
  typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
  short4_t qa[KS];
  bf16x8_t qa8[W32 ? D / 32 : 1];
  {
    const int64_t t = t0 + lr;
    const bf16* qrow = q + (((int64_t)b * s.T + (t < s.T ? t : 0)) * s.Hq + h) * D;
    if constexpr (W32) {
#pragma unroll
      for (int kb = 0; kb < D / 32; ++kb) {
        const uint4 v = t < s.T ? *(const uint4*)(qrow + kb * 32 + 8 * lq) : make_uint4(0, 0, 0, 0);
        qa8[kb] = __builtin_bit_cast(bf16x8_t, v);
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < KS; ++kb) {
        const uint2 v = t < s.T ? *(const uint2*)(qrow + kb * 16 + 4 * lq) : make_uint2(0, 0);
        qa[kb] = __builtin_bit_cast(short4_t, v);
      }
    }
  }
  float4_t o[KS];
#pragma unroll
  for (int dn = 0; dn < KS; ++dn) o[dn] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m[1] = {-__builtin_inff()}, lsum[1] = {0.f};  // of this lane's query (t0 + lr), base 2
  const int64_t tb_last = std::min<int64_t>((int64_t)blockIdx.y * PQ + PQ - 1, s.T - 1);
  const int64_t key_end = cache_len + tb_last + 1;  // keys the block's queries may see

  // Tile staging: thread t owns KQ consecutive keys of one 16-byte column pc
  // (t = kq * PPRW + pc). Its K pieces go to LDS as they are; its V pieces are
  // transposed on the way, KQ keys of one dim packed into one LDS write. The
  // next tile's pieces are loaded into registers while the current tile is
  // computed. Buffer loads past key_end read zeros (no branch, no wait).
  constexpr int NPC = KT * PPRW;                // 16-byte pieces per matrix per tile
  constexpr int KQ = NPC >= PW * 64 ? NPC / (PW * 64) : 1;
  const int kq = tid / PPRW, pc = tid % PPRW;
  // V by key-consecutive lanes: the transposed writes of one dim by 16 lanes
  // fill one contiguous run of a Vt row (no bank conflicts)
  const int kqv = tid % (KT / KQ), pcv = tid / (KT / KQ);
  const bool stager = tid < NPC / KQ;
  const uint32_t kv_bytes = (uint32_t)(key_end * D * 2);
  const __amdgpu_buffer_rsrc_t krs = span_rsrc(kbase, kv_bytes), vrs = span_rsrc(vbase, kv_bytes);
  uint4 kr[KQ], vr[KQ];
  auto load_tile = [&](int64_t k0) {
#pragma unroll
    for (int u = 0; u < KQ; ++u) {
      const int64_t key = k0 + kq * KQ + u, keyv = k0 + kqv * KQ + u;
      kr[u] = attn_load16(krs, stager && key < key_end ? (uint32_t)((key * D + pc * 8) * 2) : kv_bytes);
      vr[u] = attn_load16(vrs, stager && keyv < key_end ? (uint32_t)((keyv * D + pcv * 8) * 2) : kv_bytes);
    }
  };
  auto store_tile = [&]() {
    if (!stager) return;
#pragma unroll
    for (int u = 0; u < KQ; ++u) *(uint4*)(Ks + (kq * KQ + u) * KROW + pc * 16) = kr[u];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint16_t hv[KQ];
#pragma unroll
      for (int u = 0; u < KQ; ++u) {
        const uint32_t wv = e < 2 ? vr[u].x : e < 4 ? vr[u].y : e < 6 ? vr[u].z : vr[u].w;
        hv[u] = (uint16_t)(e & 1 ? wv >> 16 : wv);
      }
      char* dst = Vt + (pcv * 8 + e) * VROW + kqv * KQ * 2;
      if constexpr (KQ == 4) {
        *(uint2*)dst = make_uint2(hv[0] | ((uint32_t)hv[1] << 16), hv[2] | ((uint32_t)hv[3] << 16));
      } else if constexpr (KQ == 2) {
        *(uint32_t*)dst = hv[0] | ((uint32_t)hv[1] << 16);
      } else {
#pragma unroll
        for (int u = 0; u < KQ; ++u) *(uint16_t*)(dst + 2 * u) = hv[u];
      }
    }
  };

  load_tile(0);
  for (int64_t k0 = 0; k0 < key_end; k0 += KT) {
    __syncthreads();  // the previous tile is consumed
    store_tile();
    __syncthreads();
    if (k0 + KT < key_end) load_tile(k0 + KT);  // in flight during this tile's math
    if (t0 >= s.T || k0 > cache_len + t0 + 15) continue;  // this strip sees none of the tile
    // ---- scores, transposed: S^T[key k0 + 16 kbk + 4 lq + i][query t0 + lr]
    // (A = the K rows, B = Q^T: the query operand registers as they are)
    const int64_t qpos = cache_len + t0 + lr;  // this lane's query position
    float sc[KB][4];
    float mx = -__builtin_inff();
#pragma unroll
    for (int kbk = 0; kbk < KB; ++kbk) {
      float4_t acc = {0.f, 0.f, 0.f, 0.f};
      const char* krow = Ks + (kbk * 16 + lr) * KROW;
      if constexpr (W32) {
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
          const bf16x8_t kv = __builtin_bit_cast(bf16x8_t, *(const uint4*)(krow + (kb * 32 + 8 * lq) * 2));
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, qa8[kb], acc, 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int kb = 0; kb < KS; ++kb) {
          const short4_t kv = *(const short4_t*)(krow + (kb * 16 + 4 * lq) * 2);
          acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(kv, qa[kb], acc, 0, 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t key = k0 + kbk * 16 + 4 * lq + i;
        sc[kbk][i] = key <= qpos ? acc[i] * sl2 : -__builtin_inff();
        mx = fmaxf(mx, sc[kbk][i]);
      }
    }
    // ---- online softmax of this lane's query (its keys sit in lanes lr, lr + 16, + 32, + 48)
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m[0], mx);
    const float alpha = mn == -__builtin_inff() ? 1.f : __builtin_amdgcn_exp2f(m[0] - mn);
    m[0] = mn;
    lsum[0] *= alpha;
#pragma unroll
    for (int dn = 0; dn < KS; ++dn)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[dn][i] *= alpha;
    // ---- O^T += V^T P^T: P^T[key 4 lq + e][query lr] is this lane's scores, as they are
    uint2 pk[KB];  // this lane's probabilities of key block kk, bf16
#pragma unroll
    for (int kk = 0; kk < KB; ++kk) {
      float pr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[i] = sc[kk][i] == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(sc[kk][i] - mn);
        lsum[0] += pr[i];
      }
      pk[kk] = make_uint2(pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]));
    }
    if constexpr (W32) {
      // one MFMA per 32 keys: k-index 8 lq + e is key 32 j + 4 lq + e (e < 4) or
      // 32 j + 16 + 4 lq + (e - 4), the same permutation in both operands
#pragma unroll
      for (int j = 0; j < KB / 2; ++j) {
        const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, make_uint4(pk[2 * j].x, pk[2 * j].y, pk[2 * j + 1].x,
                                                                    pk[2 * j + 1].y));
#pragma unroll
        for (int dn = 0; dn < KS; ++dn) {
          const char* vrow = Vt + (dn * 16 + lr) * VROW;
          const uint2 v0 = *(const uint2*)(vrow + (32 * j + 4 * lq) * 2);
          const uint2 v1 = *(const uint2*)(vrow + (32 * j + 16 + 4 * lq) * 2);
          const bf16x8_t va = __builtin_bit_cast(bf16x8_t, make_uint4(v0.x, v0.y, v1.x, v1.y));
          o[dn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, o[dn], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < KB; ++kk) {
        const short4_t pb = __builtin_bit_cast(short4_t, pk[kk]);
#pragma unroll
        for (int dn = 0; dn < KS; ++dn) {
          const short4_t va = *(const short4_t*)(Vt + (dn * 16 + lr) * VROW + (kk * 16 + 4 * lq) * 2);
          o[dn] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb, o[dn], 0, 0, 0);
        }
      }
    }
  }
  if (t0 >= s.T) return;
  // row sum of this lane's query over the four lanes holding its keys
  float l = lsum[0];
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  const int64_t t = t0 + lr;
  if (t >= s.T) return;
  bf16* orow = out + (((int64_t)b * s.T + t) * s.Hq + h) * D;
#pragma unroll
  for (int dn = 0; dn < KS; ++dn)  // O^T[dim 16 dn + 4 lq + i][query lr]: four consecutive dims
    *(uint2*)(orow + dn * 16 + 4 * lq) =
        make_uint2(pack_bf16x2(o[dn][0] / l, o[dn][1] / l), pack_bf16x2(o[dn][2] / l, o[dn][3] / l));
}

// Maximum / sum over lanes l, l ^ 16, l ^ 32, l ^ 48 on gfx950's permlane
// swaps (VALU, no LDS round trip): with both operands equal, a 16-swap leaves
// lane l's value in one result and lane l ^ 16's in the other, a 32-swap
// likewise for l ^ 32.
__device__ __forceinline__ float quad_rows_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float quad_rows_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Long-prompt prefill on matrix cores (bf16, D % 32 == 0). Block = one
// 128-query tile of one head; its four waves own 32 queries each, as two
// 16-query strips that share every K and V operand read from LDS (half the
// LDS traffic of one strip per wave). Products transposed as in
// prefill_attn_mfma_kernel (S^T = K Q^T, O^T = V^T P^T, 16x16x32 MFMA), with
//  * K / V tiles of 64 keys double-buffered in LDS: one barrier per tile, the
//    next tile's global loads in flight during the current tile's math;
//  * the causal mask applied only on tiles that cross a query of the wave,
//    the 1/sqrt(D) scale folded into the exponent (exp2(s * c - m)), and the
//    running-sum / output rescale skipped when no lane's maximum moved;
//  * query tiles dispatched last (longest) first, and the heads of one KV
//    group kept on one XCD when the head count allows (blocks go to the
//    eight XCDs round-robin by linear id, and each XCD has its own L2).
template <int D>
__global__ __launch_bounds__(256, 2) void prefill_attn_fa_kernel(const bf16* q, const bf16* kc, const bf16* vc, bf16* out,
                                                              AttnShape s, int64_t cache_len, float scale,
                                                              PrefillKV kv) {
  kv.resolve(kc, vc, cache_len);
  typedef float float4_t __attribute__((ext_vector_type(4)));
  typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
  constexpr int NS = 2;              // 16-query strips per wave
  constexpr float RESCALE_SLACK = 8.f;
  constexpr int PQ = 4 * 16 * NS;    // queries per block
  constexpr int KT = 64, KB = KT / 16, KS = D / 16, D32 = D / 32, PPRW = D / 8;
  constexpr int KROW = D * 2 + 16, VROW = KT * 2 + 8;
  constexpr int KBYTES = KT * KROW, STAGE = KBYTES + D * VROW;
  __shared__ __attribute__((aligned(16))) char lds[2 * STAGE];
  const int G = s.Hq / s.Hkv;
  int bh = blockIdx.x;
  if (gridDim.x % 8 == 0) bh = (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8;  // XCD c: a run of heads
  const int b = bh / s.Hq, h = bh % s.Hq, g = h / G;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane % 16, lq = lane / 16;
  const int64_t qt = (int64_t)gridDim.y - 1 - blockIdx.y;
  const int64_t tw = qt * PQ + wave * 16 * NS;  // first query of this wave
  const bf16* kbase = kc + ((int64_t)b * s.Hkv + g) * s.S * D;
  const bf16* vbase = vc + ((int64_t)b * s.Hkv + g) * s.S * D;
  const float sl2 = scale * 1.4426950408889634f;

  bf16x8_t qa[NS][D32];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const int64_t t = tw + 16 * st + lr;
    const bf16* qrow = q + (((int64_t)b * s.T + (t < s.T ? t : 0)) * s.Hq + h) * D;
#pragma unroll
    for (int kb = 0; kb < D32; ++kb) {
      const uint4 v = t < s.T ? *(const uint4*)(qrow + kb * 32 + 8 * lq) : make_uint4(0, 0, 0, 0);
      qa[st][kb] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  float4_t o[NS][KS];
  float m[NS], lsum[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    m[st] = -__builtin_inff();
    lsum[st] = 0.f;
#pragma unroll
    for (int dn = 0; dn < KS; ++dn) o[st][dn] = float4_t{0.f, 0.f, 0.f, 0.f};
  }
  const int64_t tb_last = std::min<int64_t>(qt * PQ + PQ - 1, s.T - 1);
  const int64_t key_end = cache_len + tb_last + 1;
  const int64_t ntiles = cdiv(key_end, (int64_t)KT);

  // Staging: a thread loads KQ keys of one 16-byte column of K and of V. K
  // columns go to consecutive lanes (whole rows per load instruction, stored
  // as they are); V keys go to consecutive lanes, so that the transposed
  // writes of one dim by 16 lanes fill one contiguous 128-byte run of a Vt row
  // (no bank conflicts), at the price of 64-byte row segments per load.
  constexpr int NPC = KT * PPRW;
  constexpr int KQ = NPC >= 256 ? NPC / 256 : 1;
  const int kq = tid / PPRW, pc = tid % PPRW;
  const int kqv = tid % (KT / KQ), pcv = tid / (KT / KQ);
  static_assert(NPC / KQ == 256, "every thread stages");
  // pieces of keys past key_end lie past the buffer's size and read as zeros
  const uint32_t kv_bytes = (uint32_t)(key_end * D * 2);
  const __amdgpu_buffer_rsrc_t krs = span_rsrc(kbase, kv_bytes), vrs = span_rsrc(vbase, kv_bytes);
  const uint32_t koff = (uint32_t)((kq * KQ * D + pc * 8) * 2), voff = (uint32_t)((kqv * KQ * D + pcv * 8) * 2);
  uint4 kr[KQ], vr[KQ];
  auto load_tile = [&](int64_t k0) {
    const uint32_t base = (uint32_t)(k0 * D * 2);
#pragma unroll
    for (int u = 0; u < KQ; ++u) {
      kr[u] = attn_load16(krs, base + koff + u * D * 2);
      vr[u] = attn_load16(vrs, base + voff + u * D * 2);
    }
  };
  auto store_tile = [&](char* Ks) {
    char* Vt = Ks + KBYTES;
#pragma unroll
    for (int u = 0; u < KQ; ++u) *(uint4*)(Ks + (kq * KQ + u) * KROW + pc * 16) = kr[u];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint16_t hv[KQ];
#pragma unroll
      for (int u = 0; u < KQ; ++u) {
        const uint32_t wv = e < 2 ? vr[u].x : e < 4 ? vr[u].y : e < 6 ? vr[u].z : vr[u].w;
        hv[u] = (uint16_t)(e & 1 ? wv >> 16 : wv);
      }
      char* dst = Vt + (pcv * 8 + e) * VROW + kqv * KQ * 2;
      if constexpr (KQ == 4) {
        *(uint2*)dst = make_uint2(hv[0] | ((uint32_t)hv[1] << 16), hv[2] | ((uint32_t)hv[3] << 16));
      } else if constexpr (KQ == 2) {
        *(uint32_t*)dst = hv[0] | ((uint32_t)hv[1] << 16);
      } else {
#pragma unroll
        for (int u = 0; u < KQ; ++u) *(uint16_t*)(dst + 2 * u) = hv[u];
      }
    }
  };

  load_tile(0);
  store_tile(lds);
  if (ntiles > 1) load_tile(KT);
  __syncthreads();
  for (int64_t it = 0; it < ntiles; ++it) {
    const int64_t k0 = it * KT;
    const char* Ks = lds + (it & 1) * STAGE;
    const char* Vt = Ks + KBYTES;
    if (tw < s.T && k0 <= cache_len + tw + 16 * NS - 1) {  // the wave sees part of the tile
      float4_t acc[NS][KB];
#pragma unroll
      for (int kbk = 0; kbk < KB; ++kbk) {
        const char* krow = Ks + (kbk * 16 + lr) * KROW;
#pragma unroll
        for (int kb = 0; kb < D32; ++kb) {
          const bf16x8_t kv = __builtin_bit_cast(bf16x8_t, *(const uint4*)(krow + (kb * 32 + 8 * lq) * 2));
#pragma unroll
          for (int st = 0; st < NS; ++st)
            acc[st][kbk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                kv, qa[st][kb], kb == 0 ? float4_t{0.f, 0.f, 0.f, 0.f} : acc[st][kbk], 0, 0, 0);
        }
      }
      if (k0 + KT - 1 > cache_len + tw) {  // some key of the tile lies past some query of the wave
        __asm__ volatile("");                // (a branch, not selects on every tile)
        // key k0 + 16 kbk + 4 lq + i is visible to query tw + 16 st + lr when
        // 16 kbk + i <= cache_len + tw - k0 + 16 st + lr - 4 lq
        const int rel = (int)(cache_len + tw - k0) + lr - 4 * lq;
#pragma unroll
        for (int st = 0; st < NS; ++st)
#pragma unroll
          for (int kbk = 0; kbk < KB; ++kbk)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (16 * kbk + i > rel + 16 * st) acc[st][kbk][i] = -__builtin_inff();
      }
      uint2 pk[NS][KB];
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        // this lane's query: its 64 keys sit in lanes lr, lr + 16, + 32, + 48. Every
        // query sees key 0 of tile 0, so the running maximum is finite from there on.
        float mx = acc[st][0][0];
#pragma unroll
        for (int kbk = 0; kbk < KB; ++kbk)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, acc[st][kbk][i]);
        mx = quad_rows_max(mx) * sl2;
        // The reference point m moves only when some lane's maximum passes it
        // by more than RESCALE_SLACK (base 2): until then the probabilities
        // exp2(s - m) stay below 2^RESCALE_SLACK, and O and the sum keep their
        // scale (the result is the same up to rounding, fewer rescales).
        if (__builtin_amdgcn_ballot_w64(mx > m[st] + RESCALE_SLACK)) {
          const float mn = fmaxf(m[st], mx);
          const float alpha = __builtin_amdgcn_exp2f(m[st] - mn);
          m[st] = mn;
          lsum[st] *= alpha;
#pragma unroll
          for (int dn = 0; dn < KS; ++dn)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[st][dn][i] *= alpha;
        }
#pragma unroll
        for (int kbk = 0; kbk < KB; ++kbk) {
          float pr[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pr[i] = __builtin_amdgcn_exp2f(fmaf(acc[st][kbk][i], sl2, -m[st]));
            lsum[st] += pr[i];
          }
          pk[st][kbk] = make_uint2(pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]));
        }
      }
      // O^T += V^T P^T, one MFMA per 32 keys (k-index 8 lq + e = key 32 j + 4 lq + e,
      // e < 4, or 32 j + 16 + 4 lq + e - 4: the same permutation in both operands)
#pragma unroll
      for (int j = 0; j < KB / 2; ++j) {
        bf16x8_t pb[NS];
#pragma unroll
        for (int st = 0; st < NS; ++st)
          pb[st] = __builtin_bit_cast(bf16x8_t, make_uint4(pk[st][2 * j].x, pk[st][2 * j].y, pk[st][2 * j + 1].x,
                                                           pk[st][2 * j + 1].y));
#pragma unroll
        for (int dn = 0; dn < KS; ++dn) {
          const char* vrow = Vt + (dn * 16 + lr) * VROW;
          const uint2 v0 = *(const uint2*)(vrow + (32 * j + 4 * lq) * 2);
          const uint2 v1 = *(const uint2*)(vrow + (32 * j + 16 + 4 * lq) * 2);
          const bf16x8_t va = __builtin_bit_cast(bf16x8_t, make_uint4(v0.x, v0.y, v1.x, v1.y));
#pragma unroll
          for (int st = 0; st < NS; ++st)
            o[st][dn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[st], o[st][dn], 0, 0, 0);
        }
      }
    }
    if (it + 1 < ntiles) store_tile(lds + ((it + 1) & 1) * STAGE);  // that buffer was last read before the previous barrier
    __syncthreads();
    if (it + 2 < ntiles) load_tile((it + 2) * KT);
  }
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const float l = quad_rows_sum(lsum[st]);
    const int64_t t = tw + 16 * st + lr;
    if (t >= s.T) continue;
    bf16* orow = out + (((int64_t)b * s.T + t) * s.Hq + h) * D;
#pragma unroll
    for (int dn = 0; dn < KS; ++dn)
      *(uint2*)(orow + dn * 16 + 4 * lq) = make_uint2(pack_bf16x2(o[st][dn][0] / l, o[st][dn][1] / l),
                                                      pack_bf16x2(o[st][dn][2] / l, o[st][dn][3] / l));
  }
}

template <typename T, int D, int HP>
int decode_launch(hipStream_t st, DecodeArgs& a, int nsplit) {
  const int G = a.s.Hq / a.s.Hkv;
  const dim3 grid(a.s.B * a.s.Hkv, nsplit, (unsigned)cdiv(G, HP));
  hipLaunchKernelGGL((decode_attn_kernel<T, D, HP>), grid, dim3(NW * 64), 0, st, a);
  MINITP_LAUNCH_CHECK();
  if (nsplit > 1) {
    const dim3 mg((unsigned)(a.s.B * a.s.Hkv), (unsigned)cdiv(a.s.Hq / a.s.Hkv * D, MERGE_T));
    hipLaunchKernelGGL((decode_merge_kernel<T, D>), mg, dim3(MERGE_T), 0, st, a, nsplit);
    MINITP_LAUNCH_CHECK();
  }
  return MINITP_OK;
}

// Heads per wave: one while (batch rows x KV heads x splits) leaves most CUs
// idle, else the whole group.
template <typename T, int D>
int decode_dispatch(hipStream_t st, DecodeArgs& a, int nsplit) {
  const int G = a.s.Hq / a.s.Hkv;
  if ((int64_t)a.s.B * a.s.Hkv * nsplit < 128 || G == 1) return decode_launch<T, D, 1>(st, a, nsplit);
  if (G == 2) return decode_launch<T, D, 2>(st, a, nsplit);
  if (G <= 4) return decode_launch<T, D, 4>(st, a, nsplit);
  return decode_launch<T, D, 8>(st, a, nsplit);
}

template <typename T>
int decode_by_d(hipStream_t st, DecodeArgs& a, int nsplit) {
  switch (a.s.D) {
    case 16:
      return decode_dispatch<T, 16>(st, a, nsplit);
    case 32:
      return decode_dispatch<T, 32>(st, a, nsplit);
    case 64:
      return decode_dispatch<T, 64>(st, a, nsplit);
    case 128:
      return decode_dispatch<T, 128>(st, a, nsplit);
  }
  set_error("attention: head_dim %d not supported (16, 32, 64, 128)", a.s.D);
  return MINITP_ERR_UNSUPPORTED;
}

template <typename T, int D>
int prefill_dispatch(hipStream_t st, const void* q, const void* k, const void* v, void* out, const AttnShape& s,
                     int64_t cache_len, const PrefillKV& kv) {
  const float scale = 1.0f / sqrtf((float)D);
  if constexpr (sizeof(T) == 2) {
    // 128-query blocks (eight strips share each staged K / V tile) once they
    // fill the chip; 64-query blocks for short prompts
    if (D % 32 == 0 && (int64_t)s.B * s.Hq * cdiv(s.T, 128) >= 512)
      hipLaunchKernelGGL((prefill_attn_fa_kernel<D % 32 == 0 ? D : 32>), dim3(s.B * s.Hq, (unsigned)cdiv(s.T, 128)),
                         dim3(256), 0, st, (const bf16*)q, (const bf16*)k, (const bf16*)v, (bf16*)out, s, cache_len,
                         scale, kv);
    else if ((int64_t)s.B * s.Hq * cdiv(s.T, 128) >= 512)
      hipLaunchKernelGGL((prefill_attn_mfma_kernel<D, 8>), dim3(s.B * s.Hq, (unsigned)cdiv(s.T, 128)), dim3(512), 0,
                         st, (const bf16*)q, (const bf16*)k, (const bf16*)v, (bf16*)out, s, cache_len, scale, kv);
    else
      hipLaunchKernelGGL((prefill_attn_mfma_kernel<D, 4>), dim3(s.B * s.Hq, (unsigned)cdiv(s.T, 64)), dim3(256), 0,
                         st, (const bf16*)q, (const bf16*)k, (const bf16*)v, (bf16*)out, s, cache_len, scale, kv);
  } else
    hipLaunchKernelGGL((prefill_attn_kernel<T, D>), dim3(s.B * s.Hq, (unsigned)cdiv(s.T, QT)), dim3(256), 0, st,
                       (const T*)q, (const T*)k, (const T*)v, (T*)out, s, cache_len, scale, kv);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

template <typename T>
int prefill_by_d(hipStream_t st, const void* q, const void* k, const void* v, void* out, const AttnShape& s,
                 int64_t cache_len, const PrefillKV& kv) {
  switch (s.D) {
    case 16:
      return prefill_dispatch<T, 16>(st, q, k, v, out, s, cache_len, kv);
    case 32:
      return prefill_dispatch<T, 32>(st, q, k, v, out, s, cache_len, kv);
    case 64:
      return prefill_dispatch<T, 64>(st, q, k, v, out, s, cache_len, kv);
    case 128:
      return prefill_dispatch<T, 128>(st, q, k, v, out, s, cache_len, kv);
  }
  set_error("attention: head_dim %d not supported (16, 32, 64, 128)", s.D);
  return MINITP_ERR_UNSUPPORTED;
}

// Blocks per (b, KV head) for contexts up to `ctx`: one while each wave has
// at most four chunks to walk, more (up to about one block per CU overall)
// beyond that. Batched decode (16 or more (b, KV head) units) splits down to
// two chunks per wave, up to about four blocks per CU: at batch 32 x 2,300
// positions (64 units, 40 chunks) that is 3 splits instead of 2, 3.8 % more
// tokens per second; one chunk per wave (5 splits) measured 8 % fewer.
// Splits of the MFMA form: about 2 blocks per CU, each wave at least two
// 32-position tiles.
#ifndef MINITP_DEC_MF_BLOCKS
#define MINITP_DEC_MF_BLOCKS 256
#endif
#ifndef MINITP_DEC_MF_TILES
#define MINITP_DEC_MF_TILES 2
#endif
int64_t decode_mfma_nsplit(int64_t units, int64_t ctx) {
  const int64_t tiles = cdiv(std::max<int64_t>(ctx, 1), 32);
  const int64_t by_tiles = std::max<int64_t>(1, tiles / (MINITP_DEC_MF_TILES * NWM));
  return std::max<int64_t>(1, std::min<int64_t>(cdiv(MINITP_DEC_MF_BLOCKS, std::max<int64_t>(units, 1)), by_tiles));
}

// The MFMA form serves bf16 groups of 2..GMAX heads at D = 64 / 128 from 16
// (rows x KV heads) up: below that the per-head blocks of decode_attn_kernel
// spread the few units wider. Measured with 2,048-token prompts: 0.5B batch
// 16 1.19 -> 0.97 ms a step and batch 24 1.27 -> 1.10 against a threshold of
// 64 units; 7B batch 4 962 -> 1,005 tokens/s; 7B batch 2 (8 units) is
// faster on the per-head kernel (535 against 511).
bool decode_use_mfma(int dtype, int64_t units, int G, int D) {
  return dtype == MINITP_BF16 && (D == 64 || D == 128) && G >= 2 && G <= GMAX && units >= 16;
}

int64_t decode_nsplit(int64_t units, int64_t ctx, int64_t D) {
  const int64_t cp = D >= 128 ? 32 : 64;
  const int64_t chunks = cdiv(std::max<int64_t>(ctx, 1), cp);
  if (units >= 16) return std::max<int64_t>(1, std::min<int64_t>(cdiv(chunks, 2 * NW), 1024 / units));
  const int64_t want = cdiv(chunks, 4 * NW);
  return std::max<int64_t>(1, std::min<int64_t>(want, std::max<int64_t>(1, 256 / std::max<int64_t>(units, 1))));
}

}  // namespace

int64_t attention_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t S) {
  (void)T;
  (void)Hq;
  const int64_t units = B * Hkv;
  const int64_t ns = std::max(decode_nsplit(units, S, D), decode_mfma_nsplit(units, S));
  return units * ns * GMAX * 2 * 4 + units * ns * GMAX * D * 4;
}

int launch_decode_attention(hipStream_t st, int dtype, const void* q, const void* k_cache, const void* v_cache,
                            void* out, const AttnShape& s, int64_t cache_len, const StepState* state, int layer,
                            void* workspace, int64_t workspace_bytes) {
  if (s.Hq % s.Hkv != 0 || s.Hq / s.Hkv > GMAX) {
    set_error("attention: Hq=%d Hkv=%d (group must divide and be <= %d)", s.Hq, s.Hkv, GMAX);
    return MINITP_ERR_UNSUPPORTED;
  }
  if (s.S * s.D * (dtype == MINITP_F32 ? 4 : 2) >= (1LL << 32)) {
    set_error("attention: a (row, KV head) cache of %lld x %d exceeds 4 GiB", (long long)s.S, s.D);
    return MINITP_ERR_UNSUPPORTED;
  }
  const int64_t need = attention_workspace_bytes(s.B, 1, s.Hq, s.Hkv, s.D, s.S);
  if (workspace_bytes < need || workspace == nullptr) {
    set_error("attention: workspace %lld B < %lld B", (long long)workspace_bytes, (long long)need);
    return MINITP_ERR_ARG;
  }
  if (s.B == 0) return MINITP_OK;
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
  // graph replays size the grid for a full cache; direct calls for this step
  const int64_t ctx = state ? s.S : cache_len + 1;
  const bool mf = decode_use_mfma(dtype, units, s.Hq / s.Hkv, s.D);
  const int nsplit = (int)(mf ? decode_mfma_nsplit(units, ctx) : decode_nsplit(units, ctx, s.D));
  a.ws_ml = (float*)workspace;
  a.ws_o = a.ws_ml + units * nsplit * GMAX * 2;
  // inside a forward: the step state's arrival words, the merge in-kernel
  a.count = state != nullptr && units <= SPLIT_MAX_TUPLES
                ? (uint32_t*)((char*)const_cast<StepState*>(state) + offsetof(StepState, split_count))
                : nullptr;
  if (mf) {
    const dim3 grid((unsigned)units, (unsigned)nsplit);
    const void* kern = s.D == 64 ? (const void*)decode_attn_mfma_kernel<64> : (const void*)decode_attn_mfma_kernel<128>;
    const int lds = NWM * (s.D == 64 ? MfDec<64>::WAVE_LDS : MfDec<128>::WAVE_LDS);
    int rc = ensure_lds_limit(kern, lds);
    if (rc) return rc;
    if (s.D == 64)
      hipLaunchKernelGGL(decode_attn_mfma_kernel<64>, grid, dim3(NWM * 64), lds, st, a);
    else
      hipLaunchKernelGGL(decode_attn_mfma_kernel<128>, grid, dim3(NWM * 64), lds, st, a);
    MINITP_LAUNCH_CHECK();
    if (nsplit > 1 && a.count == nullptr) {
      const dim3 mg((unsigned)units, (unsigned)cdiv(s.Hq / s.Hkv * s.D, MERGE_T));
      if (s.D == 64)
        hipLaunchKernelGGL((decode_merge_kernel<bf16, 64>), mg, dim3(MERGE_T), 0, st, a, nsplit);
      else
        hipLaunchKernelGGL((decode_merge_kernel<bf16, 128>), mg, dim3(MERGE_T), 0, st, a, nsplit);
      MINITP_LAUNCH_CHECK();
    }
    return MINITP_OK;
  }
  return dtype == MINITP_F32 ? decode_by_d<float>(st, a, nsplit) : decode_by_d<bf16>(st, a, nsplit);
}

// The folded o_proj: one batch row, one KV group per block row of heads,
// head dims with whole 16-byte chunks, and a W_o slice of at most 16 loads
// per thread in at most OPROJ_MAX_SLICES slices (more would re-run each
// head's attention too often).
constexpr int OPROJ_MAX_SLICES = 16;
constexpr int OPROJ_MAX_NLW = 16;

int attn_oproj_rows(int dtype, const AttnShape& s, int64_t H, int slices) {
  const int es = dtype == MINITP_F32 ? 4 : 2;
  const int64_t cpr = (int64_t)s.D * es / 16;  // loads per row segment
  const int64_t per_block = (int64_t)OPROJ_MAX_NLW * NW * 64 / std::max<int64_t>(cpr, 1);
  const int64_t rows = std::max<int64_t>(cdiv(H, std::max(slices, 1)), 1);
  return (int)std::min<int64_t>(per_block, rows);
}

bool attn_oproj_supported(int dtype, const AttnShape& s, int64_t H, int slices) {
  if (s.B != 1 || s.T != 1 || s.Hkv < 1 || s.Hq % s.Hkv != 0 || s.Hq / s.Hkv > GMAX || H < 1) return false;
  if (!(s.D == 16 || s.D == 32 || s.D == 64 || s.D == 128) || s.Hq > PART_MAX_PARTS) return false;
  const int es = dtype == MINITP_F32 ? 4 : 2;
  if (s.S * s.D * es >= (1LL << 32)) return false;
  if ((int64_t)s.D * es % 16 != 0 || (int64_t)s.D * es / 16 > 64) return false;
  const int rows = attn_oproj_rows(dtype, s, H, slices);
  return cdiv(H, rows) <= OPROJ_MAX_SLICES && (int64_t)rows * s.Hq * s.D * es < (1LL << 31);
}

namespace {
template <typename T, int D, int NLW>
void oproj_launch(hipStream_t st, DecodeArgs& a, dim3 grid) {
  hipLaunchKernelGGL((decode_attn_kernel<T, D, 1, NLW>), grid, dim3(NW * 64), 0, st, a);
}

template <typename T, int D>
int oproj_by_nlw(hipStream_t st, DecodeArgs& a) {
  const int cpr = D * (int)sizeof(T) / 16;
  const int64_t chunks = (int64_t)a.op.rows * cpr;
  const dim3 grid((unsigned)a.s.Hkv, (unsigned)cdiv(a.op.H, a.op.rows), (unsigned)(a.s.Hq / a.s.Hkv));
  if (chunks <= NW * 64)
    oproj_launch<T, D, 1>(st, a, grid);
  else if (chunks <= 2 * NW * 64)
    oproj_launch<T, D, 2>(st, a, grid);
  else if (chunks <= 4 * NW * 64)
    oproj_launch<T, D, 4>(st, a, grid);
  else if (chunks <= 8 * NW * 64)
    oproj_launch<T, D, 8>(st, a, grid);
  else
    oproj_launch<T, D, 16>(st, a, grid);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

template <typename T>
int oproj_by_d(hipStream_t st, DecodeArgs& a) {
  switch (a.s.D) {
    case 16:
      return oproj_by_nlw<T, 16>(st, a);
    case 32:
      return oproj_by_nlw<T, 32>(st, a);
    case 64:
      return oproj_by_nlw<T, 64>(st, a);
    default:
      return oproj_by_nlw<T, 128>(st, a);
  }
}
}  // namespace

int launch_decode_attention_oproj(hipStream_t st, int dtype, const void* q, const AttnShape& s,
                                  const StepState* state, int layer, const OprojArgs& o) {
  const int slices = (int)cdiv(o.H, std::max(o.rows, 1));
  if (!attn_oproj_supported(dtype, s, o.H, slices) || state == nullptr ||
      o.rows != attn_oproj_rows(dtype, s, o.H, slices) || !aligned16(o.w) || o.part == nullptr) {
    set_error("attention + o_proj: unsupported shape (B=%d T=%d Hq=%d Hkv=%d D=%d H=%lld)", s.B, s.T, s.Hq, s.Hkv,
              s.D, (long long)o.H);
    return MINITP_ERR_UNSUPPORTED;
  }
  DecodeArgs a{};
  a.q = q;
  a.s = s;
  a.st = state;
  a.layer = layer;
  a.scale = 1.0f / sqrtf((float)s.D);
  a.op = o;
  return dtype == MINITP_F32 ? oproj_by_d<float>(st, a) : oproj_by_d<bf16>(st, a);
}

int launch_prefill_attention(hipStream_t st, int dtype, const void* q, const void* k_cache, const void* v_cache,
                             void* out, const AttnShape& s, int64_t cache_len, const StepState* state, int layer) {
  const PrefillKV kv{state, (int64_t)layer * s.B * s.Hkv * s.S * s.D};
  if (s.Hq % s.Hkv != 0) {
    set_error("attention: Hq=%d not divisible by Hkv=%d", s.Hq, s.Hkv);
    return MINITP_ERR_ARG;
  }
  if (s.B * s.T == 0) return MINITP_OK;
  return dtype == MINITP_F32 ? prefill_by_d<float>(st, q, k_cache, v_cache, out, s, cache_len, kv)
                             : prefill_by_d<bf16>(st, q, k_cache, v_cache, out, s, cache_len, kv);
}

}  // namespace minitp
