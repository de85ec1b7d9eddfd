// Decode GEMV: y = epilogue(x W^T) for M <= 4 input rows, streaming W once.
//
// Mapping (wave64, 256-thread blocks = 4 waves):
//  * Work unit = a "tuple" of 2P weight rows, P pairs (row_a + p, row_b + p).
//    The pairing lets an epilogue see two rows at once: SwiGLU pairs gate
//    row j with up row I + j (mlp.py:38), RoPE pairs head dims i and
//    i + D/2 (rope.py:57-62); plain stores use 2P contiguous rows.
//  * KSPLIT waves of a block share one tuple and split K; a block holds
//    4 / KSPLIT tuples and walks the tuple space with a grid stride.
//  * Lane l of K-split wave kw owns the 16-byte chunks c = kw*64 + l +
//    j*64*KSPLIT of every row: consecutive lanes read consecutive 16 B, so a
//    wave-load is one contiguous 1 KiB of a row.
//
// gemv_reg_kernel (rows up to 1024 chunks of 16 B, i.e. K <= 8192 bf16) is
// built for latency, which is what decode at these sizes is bound by: the
// first tuple's weight loads are issued before anything else; the input
// row(s), the RMSNorm weight and the epilogue's side inputs (RoPE table
// entries, residual) load underneath them; the input stays in registers (no
// LDS staging, no barrier unless K is split across waves); and each tuple
// prefetches the next tuple's weights before its own reduction and epilogue.
// gemv_lds_kernel stages the input in LDS and serves longer rows.
// gemv_mfma_kernel serves bf16 decode batches of 5 to 32 rows on MFMA.
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace minitp {

static int device_cus();

namespace {

constexpr int P = 2;  // pairs per tuple (R = 4 rows)
constexpr int R = 2 * P;
constexpr int U = 2;  // gemv_lds_kernel chunk unroll
constexpr int MAX_GRID = 2048;
constexpr int64_t REG_MAX_CHUNKS = 1024;
// Split-K form: chunks per lane and row in one segment, and the row length
// (in 16-byte chunks) above which single-row products take it.
#ifndef MINITP_SPLIT_JMAX
#define MINITP_SPLIT_JMAX 3
#endif
#ifndef MINITP_SPLIT_MIN_CHUNKS
#define MINITP_SPLIT_MIN_CHUNKS 1024
#endif
constexpr int SPLIT_JMAX = MINITP_SPLIT_JMAX;
constexpr int64_t SPLIT_MIN_CHUNKS = MINITP_SPLIT_MIN_CHUNKS;

// EPI_QKV_ROPE of a single-token forward: the RoPE rows come from the
// StepState, so the epilogue's side inputs need no position load first.
constexpr int EPI_QKV_ROPE1 = 5;
template <int EPI>
constexpr bool is_qkv() {
  return EPI == EPI_QKV_ROPE || EPI == EPI_QKV_ROPE1;
}

// The register path issues every input and weight load through span_rsrc
// resources, unconditionally.

// Cache-policy bits of the weight loads: nt (read once per step) when
// MINITP_NT_LOADS is set.
constexpr int W_AUX = MINITP_NT_LOADS ? 2 : 0;
// The MFMA GEMVs (3-32 input rows) load their weights non-temporal up to
// MINITP_MF_PLAIN_ROWS input rows and plain above (the half-row form, which
// serves more than 16 rows, and the SwiGLU tuple loop), except the split-K
// form and the plain-store tuple loop (the LM head), non-temporal at every
// row count. 0.5B, 2,048-token prompts, ms a step with all of them
// non-temporal / plain: batch 3 0.909 / 0.958, 4 0.905 / 0.973, 8 0.903 /
// 0.927, 16 0.960 / 0.958, 32 1.040-1.042 / 1.035-1.037; 7B batch 3-8 the
// same either way. At batch 32, the split-K form non-temporal with the
// others plain: 1.033-1.035 against 1.037-1.044 ms.
#ifndef MINITP_MF_PLAIN_ROWS
#define MINITP_MF_PLAIN_ROWS 16
#endif
constexpr int AUX_NT = 2;  // buffer-op cache policy: non-temporal
template <int AUX>
__device__ __forceinline__ uint4 span_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
  return make_uint4(v.x, v.y, v.z, v.w);
}


template <int EPI, int PP = P>
__device__ __forceinline__ void tuple_rows(int64_t t, const GemvArgs& a, int64_t& ra, int64_t& rb) {
  if constexpr (EPI == EPI_SWIGLU) {
    ra = t * PP;
    rb = a.N + t * PP;
  } else if constexpr (is_qkv<EPI>()) {
    const int half = a.a.D / 2;
    const int per_head = half / PP;
    const int t32 = (int)t;  // tuple and row indices fit 32 bits: 32-bit division
    ra = (int64_t)(t32 / per_head) * a.a.D + (t32 % per_head) * PP;
    rb = ra + half;
  } else {
    ra = t * 2 * PP;
    rb = t * 2 * PP + PP;
  }
}

template <int EPI, int PP = P>
__host__ __device__ __forceinline__ int64_t num_tuples(const GemvArgs& a) {
  if constexpr (EPI == EPI_SWIGLU) return a.N / PP;
  if constexpr (is_qkv<EPI>()) return (int64_t)(a.a.Hq + 2 * a.a.Hkv) * (a.a.D / 2) / PP;
  return cdiv(a.N, 2 * PP);
}

// Rows that exist in the weight matrix (contiguous tuples can overhang N).
template <int EPI>
__device__ __forceinline__ bool row_valid(int64_t r, const GemvArgs& a) {
  if constexpr (EPI == EPI_STORE || EPI == EPI_RESID || EPI == EPI_ARGMAX) return r < a.N;
  return true;
}

// acc += <w chunk, x chunk> for one 16-byte chunk: fp32 FMAs, or for bf16
// the packed-pair dot product v_dot2_f32_bf16 (fp32 accumulate).
template <typename T>
__device__ __forceinline__ float dot_chunk(const uint4& w, const float* xf, const uint4& xb, float acc);
template <>
__device__ __forceinline__ float dot_chunk<float>(const uint4& w, const float* xf, const uint4&, float acc) {
  acc = fmaf(__uint_as_float(w.x), xf[0], acc);
  acc = fmaf(__uint_as_float(w.y), xf[1], acc);
  acc = fmaf(__uint_as_float(w.z), xf[2], acc);
  return fmaf(__uint_as_float(w.w), xf[3], acc);
}
template <>
__device__ __forceinline__ float dot_chunk<bf16>(const uint4& w, const float*, const uint4& xb, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.x), __builtin_bit_cast(bf16x2_t, xb.x), acc,
                                        false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.y), __builtin_bit_cast(bf16x2_t, xb.y), acc,
                                        false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.z), __builtin_bit_cast(bf16x2_t, xb.z), acc,
                                        false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.w), __builtin_bit_cast(bf16x2_t, xb.w), acc,
                                         false);
}

__device__ __forceinline__ uint4 pack_bf16x8(const float* f) {
  uint4 r;
  r.x = pack_bf16x2(f[0], f[1]);
  r.y = pack_bf16x2(f[2], f[3]);
  r.z = pack_bf16x2(f[4], f[5]);
  r.w = pack_bf16x2(f[6], f[7]);
  return r;
}

// Epilogue side inputs a lane needs for pair ep of row em of tuple rows[]:
// RoPE: cos/sin of both rows (single-token forwards read the rows the first
// kernel copied into the StepState) in side[0..3] and the two bias values in
// side[4..5]; RESID: both residual values. The single-token RoPE and the
// residual loads are unconditional (clamped to rows that exist), so nothing
// has to wait for them before the epilogue.
template <typename T, int EPI, int PP = P>
__device__ __forceinline__ void load_side(const GemvArgs& a, int em, int ep, const int64_t* rows, const bool* rok,
                                          int64_t pos, float* side) {
  if constexpr (EPI == EPI_QKV_ROPE1) {
    const int D = a.a.D;
    const int i = (int)rows[ep] % D;
    side[0] = a.st->rope_cos[i];
    side[1] = a.st->rope_sin[i];
    side[2] = a.st->rope_cos[i + D / 2];
    side[3] = a.st->rope_sin[i + D / 2];
    side[4] = load_f32<T>((const T*)a.bias, rows[ep]);
    side[5] = load_f32<T>((const T*)a.bias, rows[PP + ep]);
  } else if constexpr (EPI == EPI_QKV_ROPE) {
    const int D = a.a.D;
    const int head = (int)rows[ep] / D;
    side[4] = load_f32<T>((const T*)a.bias, rows[ep]);
    side[5] = load_f32<T>((const T*)a.bias, rows[PP + ep]);
    if (head < a.a.Hq + a.a.Hkv) {
      const int i = (int)rows[ep] % D;
      if (pos >= 0 && pos < a.max_pos) {
        side[0] = a.cos_tab[pos * D + i];
        side[1] = a.sin_tab[pos * D + i];
        side[2] = a.cos_tab[pos * D + i + D / 2];
        side[3] = a.sin_tab[pos * D + i + D / 2];
      }
    }
  } else if constexpr (EPI == EPI_RESID) {
    const T* aux = (const T*)a.aux;
    const int64_t m = em < a.M ? em : 0;
    side[0] = load_f32<T>(aux, m * a.ldy + (rok[ep] ? rows[ep] : 0));
    side[1] = load_f32<T>(aux, m * a.ldy + (rok[PP + ep] ? rows[PP + ep] : 0));
  }
}

// Epilogue of one (row m, pair) for the non-argmax epilogues.
template <typename T, int EPI>
__device__ __forceinline__ void finish_pair(const GemvArgs& a, int m, int64_t row_a, int64_t row_b, bool oka,
                                            bool okb, float va, float vb, const float* side, int64_t pos) {
  if constexpr (EPI == EPI_STORE) {
    // no output pointer: the step's logits buffer (the LM head in a forward)
    T* y = (T*)(a.y != nullptr ? a.y : a.st->args.logits);
    const T* bias = (const T*)a.bias;
    if (oka) store_f32<T>(y, m * a.ldy + row_a, va + (bias ? load_f32<T>(bias, row_a) : 0.f));
    if (okb) store_f32<T>(y, m * a.ldy + row_b, vb + (bias ? load_f32<T>(bias, row_b) : 0.f));
  } else if constexpr (EPI == EPI_RESID) {
    T* y = (T*)a.y;
    if (oka) store_f32<T>(y, m * a.ldy + row_a, add_rn(side[0], round_to<T>(va)));
    if (okb) store_f32<T>(y, m * a.ldy + row_b, add_rn(side[1], round_to<T>(vb)));
  } else if constexpr (EPI == EPI_SWIGLU) {
    store_f32<T>((T*)a.y, m * a.ldy + row_a, swiglu<T>(round_to<T>(va), round_to<T>(vb)));
  } else if constexpr (is_qkv<EPI>()) {
    // F.linear output with bias, rounded to the dtype (fused.py:58)
    va = round_to<T>(va + side[4]);
    vb = round_to<T>(vb + side[5]);
    const StepState* st = a.st;
    const AttnShape& s = a.a;
    const int D = s.D, half = D / 2;
    const int head = (int)row_a / D;
    const int i = (int)row_a % D;
    const int b = m / s.T, tt = m % s.T;
    if (head < s.Hq + s.Hkv) {
      // rotate(x) = x * cos + rotate_half(x) * sin in fp32, each multiply
      // and the add rounded separately, then cast (rope.py:61-62)
      float oa, ob;
      if (s.T > 1 && (pos < 0 || pos >= a.max_pos)) {
        oa = ob = __builtin_nanf("");
        ((StepState*)st)->error = 1;
      } else {
        oa = add_rn(mul_rn(va, side[0]), -mul_rn(vb, side[1]));
        ob = add_rn(mul_rn(vb, side[2]), mul_rn(va, side[3]));
      }
      if (head < s.Hq) {
        T* q = (T*)a.y;  // [B, T, Hq, D]
        const int64_t base = ((int64_t)m * s.Hq + head) * D;
        store_f32<T>(q, base + i, oa);
        store_f32<T>(q, base + i + half, ob);
      } else if (!st->halted) {
        T* kc = (T*)st->args.k_cache + (int64_t)a.layer * s.B * s.Hkv * s.S * D;
        const int64_t base = (((int64_t)b * s.Hkv + (head - s.Hq)) * s.S + st->args.cache_len + tt) * D;
        store_f32<T>(kc, base + i, oa);
        store_f32<T>(kc, base + i + half, ob);
      }
    } else if (!st->halted) {
      T* vc = (T*)st->args.v_cache + (int64_t)a.layer * s.B * s.Hkv * s.S * D;
      const int64_t base = (((int64_t)b * s.Hkv + (head - s.Hq - s.Hkv)) * s.S + st->args.cache_len + tt) * D;
      store_f32<T>(vc, base + i, va);
      store_f32<T>(vc, base + i + half, vb);
    }
  }
}

// LM-head argmax: each block publishes its best (value, index) per row into
// part_val / part_idx [m][block]; argmax_merge_kernel (a separate launch)
// picks the winner. The order of a (value, index) comparison under
// argmax_better is total, so the merge order cannot change the winner.
// (A merge by the grid's last block, after device-coherent partial stores
// and an arrival count, measured no faster: 0.5218 against 0.5198 ms a
// token at 0.5B; the count and the partial loads cost what the launch did.)
template <int MM, int SLOTS>
__device__ __forceinline__ void argmax_finish(const GemvArgs& a, int M, int slot, int kw, const float* bv,
                                              const int64_t* bi, float (*best_v)[MM], int64_t (*best_i)[MM]) {
  const int tid = threadIdx.x, lane = tid & 63;
  if (kw == 0 && lane == 0) {
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      best_v[slot][m] = bv[m];
      best_i[slot][m] = bi[m];
    }
  }
  __syncthreads();
  if (tid < M) {
    const int m = tid;
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
}

// Chunk (V elements) of a row staged in LDS as floats, packed as the dtype's
// 16 bytes (exact: the values are already rounded to the dtype).
template <typename T>
__device__ __forceinline__ uint4 lds_chunk16(const float* xs, int64_t c) {
  if constexpr (sizeof(T) == 2) {
    return pack_bf16x8(xs + c * 8);
  } else {
    return make_uint4(__float_as_uint(xs[c * 4]), __float_as_uint(xs[c * 4 + 1]), __float_as_uint(xs[c * 4 + 2]),
                      __float_as_uint(xs[c * 4 + 3]));
  }
}

template <typename T, int MM, int KSPLIT, int JMAX, int PRO, int EPI, int PP = P>
__global__ __launch_bounds__(256) void gemv_reg_kernel(GemvArgs a) {
  // PP pairs (2 PP rows) a tuple: the names P and R below are this kernel's
  constexpr int P = PP, R = 2 * PP;
  constexpr int V = Vec<T>::N;
  constexpr int SLOTS = 4 / KSPLIT;
  constexpr bool NORM = PRO != PRO_NONE;
  constexpr bool PART = PRO == PRO_PART_NORM;
  static_assert(!PART || MM == 1, "the partial-sum prologue serves one row");
  __shared__ float red[4][MM * R];
  __shared__ float nrm[4][MM];
  __shared__ float best_v[4][MM];
  __shared__ int64_t best_i[4][MM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kw = wave % KSPLIT, slot = wave / KSPLIT;
  const int M = (int)a.M;
  const int64_t nchunk = a.K / V;
  const int64_t ntup = num_tuples<EPI, PP>(a);
  const int64_t tstride = (int64_t)gridDim.x * SLOTS;
  const uint4* W = (const uint4*)a.w;
  const uint32_t row_bytes = (uint32_t)(a.K * (int64_t)sizeof(T));

  // Load order matters: vector loads retire in issue order, so what the
  // prologue consumes (input rows, RMSNorm weight) is requested first, then
  // the epilogue's side inputs and the weights; the norm math overlaps the
  // loads still in flight. Lane l's 16-byte chunk j of a row sits at
  // byte offset (kw * 64 + l + j * 64 * KSPLIT) * 16; chunks past the row end
  // read zeros.
  int64_t t = (int64_t)blockIdx.x * SLOTS + slot;
  int64_t rows[R];
  bool rok[R];
  uint4 wv[JMAX][R];
  auto set_rows = [&](int64_t tt) {
    int64_t ra = 0, rb = 0;
    const bool ok = tt < ntup;
    if (ok) tuple_rows<EPI, PP>(tt, a, ra, rb);
#pragma unroll
    for (int p = 0; p < P; ++p) {
      rows[p] = ra + p;
      rows[P + p] = rb + p;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) rok[r] = ok && row_valid<EPI>(rows[r], a);
  };
  uint32_t coff[JMAX];
#pragma unroll
  for (int j = 0; j < JMAX; ++j) coff[j] = (uint32_t)((kw * 64 + lane + j * 64 * KSPLIT) * 16);
  auto load_w = [&]() {
    __amdgpu_buffer_rsrc_t rs[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rs[r] = span_rsrc(W + (rok[r] ? rows[r] : 0) * nchunk, rok[r] ? row_bytes : 0u);
#pragma unroll
    for (int j = 0; j < JMAX; ++j)
#pragma unroll
      for (int r = 0; r < R; ++r) wv[j][r] = span_load16<W_AUX>(rs[r], coff[j]);
  };
  set_rows(t);

  // ---- 1. input rows and RMSNorm weight ---------------------------------------
  const T* x = (const T*)a.x;
  float xf[MM][JMAX][V];
  uint4 xb[MM][JMAX];
  uint4 nw[JMAX];
  // PRO_PART_NORM: thread tid sums elements 4 tid .. 4 tid + 3 of the partial
  // rows (all of them in flight at once; rows past nparts read zeros). They
  // are requested before the weights: the prologue's sum, LDS exchange and
  // norm then overlap the weight stream (weights first measured 0.540
  // against 0.517 ms a token at 0.5B).
  u32x4 pv[PART ? PART_MAX_PARTS : 1];
  float xres[4];
  auto load_parts = [&]() {
    const __amdgpu_buffer_rsrc_t pr = span_rsrc(a.part, (uint32_t)(a.nparts * a.K * 4));
#pragma unroll
    for (int h = 0; h < PART_MAX_PARTS; ++h)
      pv[h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            pr, (uint32_t)((h * a.K + 4 * threadIdx.x) * 4), 0, 0));
    const __amdgpu_buffer_rsrc_t xr = span_rsrc(x, row_bytes);
    if constexpr (sizeof(T) == 2) {
      const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(xr, 8 * threadIdx.x, 0, 0));
      xres[0] = __uint_as_float(v.x << 16);
      xres[1] = __uint_as_float(v.x & 0xffff0000u);
      xres[2] = __uint_as_float(v.y << 16);
      xres[3] = __uint_as_float(v.y & 0xffff0000u);
    } else {
      const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, 16 * threadIdx.x, 0, 0));
      xres[0] = __uint_as_float(v.x);
      xres[1] = __uint_as_float(v.y);
      xres[2] = __uint_as_float(v.z);
      xres[3] = __uint_as_float(v.w);
    }
  };
  if constexpr (PART) load_parts();
  {
    __amdgpu_buffer_rsrc_t nr = span_rsrc(a.norm_w, NORM ? row_bytes : 0u);
#pragma unroll
    for (int j = 0; j < JMAX; ++j) nw[j] = NORM ? span_load16<0>(nr, coff[j]) : make_uint4(0, 0, 0, 0);
    if constexpr (!PART) {
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        __amdgpu_buffer_rsrc_t xr = span_rsrc(x + (m < M ? m : 0) * a.ldx, m < M ? row_bytes : 0u);
#pragma unroll
        for (int j = 0; j < JMAX; ++j) xb[m][j] = span_load16<0>(xr, coff[j]);
      }
    }
  }

  // ---- 2. the first tuple's side inputs and weights ----------------------------
  // Side inputs that need no loaded value first (the single-token RoPE rows,
  // the bias, the residual): issued here, ahead of the prologue math, they
  // arrive with the weights instead of a round trip after the norm. The
  // multi-token RoPE reads its position first, so it follows the weights.
  const int em = lane / P, ep = lane % P;  // this lane finishes pair ep of row em
  float side[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t pos = 0;
  if constexpr (EPI != EPI_QKV_ROPE) load_side<T, EPI, PP>(a, em, ep, rows, rok, pos, side);
  load_w();
  // Keep the scheduler from sinking the weight loads below the prologue math
  // (and the waits for the input rows that math needs).
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (EPI == EPI_QKV_ROPE) {
    if (em < M && a.a.T > 1) pos = a.st->args.positions[em % a.a.T];
    if (em < M && t < ntup) load_side<T, EPI, PP>(a, em, ep, rows, rok, pos, side);
  }

  // ---- 3b. PRO_PART_NORM: x + sum of the partials (in row order) ------------
  // rounded like o_proj's output and the residual add (layer.py:63), through
  // LDS to the waves' chunks; block 0 also stores the row for the residual
  // add that follows the next product
  if constexpr (PART) {
    __shared__ __attribute__((aligned(16))) float xs[PART_MAX_K];
    const int64_t e0 = 4 * (int64_t)threadIdx.x;
    if (e0 < a.K) {
      float sum[4] = {__uint_as_float(pv[0].x), __uint_as_float(pv[0].y), __uint_as_float(pv[0].z),
                      __uint_as_float(pv[0].w)};
#pragma unroll
      for (int h = 1; h < PART_MAX_PARTS; ++h) {
        if (h < a.nparts) {
          sum[0] = add_rn(sum[0], __uint_as_float(pv[h].x));
          sum[1] = add_rn(sum[1], __uint_as_float(pv[h].y));
          sum[2] = add_rn(sum[2], __uint_as_float(pv[h].z));
          sum[3] = add_rn(sum[3], __uint_as_float(pv[h].w));
        }
      }
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = round_to<T>(add_rn(xres[e], round_to<T>(sum[e])));
      *(float4*)(xs + e0) = make_float4(v[0], v[1], v[2], v[3]);  // one LDS write
      if (blockIdx.x == 0) {
        T* xo = (T*)a.x_out;
#pragma unroll
        for (int e = 0; e < 4; ++e) store_f32<T>(xo, e0 + e, v[e]);
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < JMAX; ++j) {
      const int64_t c = coff[j] / 16;
      xb[0][j] = c * V < a.K ? lds_chunk16<T>(xs, c) : make_uint4(0, 0, 0, 0);
    }
  }

  // ---- 4. input rows in registers (normed and rounded like layer.py:39-42) --
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int j = 0; j < JMAX; ++j) unpack16(xb[m][j], xf[m][j], (T*)nullptr);
  if constexpr (NORM) {
    // Every wave recomputes the row's norm, so this stays short: for bf16 the
    // sum of squares runs on packed dot instructions (exact products, fp32
    // accumulation) and the normed row is rounded two elements per
    // instruction straight into the packed operand of the dots.
    float tot[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float ss = 0.f;
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int j = 0; j < JMAX; ++j) ss = dot_chunk<T>(xb[m][j], nullptr, xb[m][j], ss);
      } else {
#pragma unroll
        for (int j = 0; j < JMAX; ++j)
#pragma unroll
          for (int e = 0; e < V; ++e) ss = add_rn(ss, mul_rn(xf[m][j][e], xf[m][j][e]));
      }
      tot[m] = wave_sum(ss);
    }
    if constexpr (KSPLIT > 1) {
      if (lane == 0)
#pragma unroll
        for (int m = 0; m < MM; ++m) nrm[wave][m] = tot[m];
      __syncthreads();
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        float s = 0.f;
        for (int k = 0; k < KSPLIT; ++k) s += nrm[slot * KSPLIT + k][m];
        tot[m] = s;
      }
    }
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(tot[m], (float)a.K), a.eps)));
#pragma unroll
      for (int j = 0; j < JMAX; ++j) {
        float wf[V];
        unpack16(nw[j], wf, (T*)nullptr);
        if constexpr (sizeof(T) == 2) {  // the dots read the packed row only
          float o[V];
#pragma unroll
          for (int e = 0; e < V; ++e) o[e] = mul_rn(mul_rn(xf[m][j][e], r), wf[e]);
          xb[m][j] = pack_bf16x8(o);
        } else {
#pragma unroll
          for (int e = 0; e < V; ++e) xf[m][j][e] = m < M ? mul_rn(mul_rn(xf[m][j][e], r), wf[e]) : 0.f;
        }
      }
    }
  }

  float bv[MM];
  int64_t bi[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    bv[m] = -__builtin_inff();
    bi[m] = INT64_MAX;
  }

  // ---- 5. tuples (grid stride), next tuple's weights prefetched -----------
  for (int64_t t0 = (int64_t)blockIdx.x * SLOTS; t0 < ntup; t0 += tstride) {
    float acc[MM][R];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < JMAX; ++j) s = dot_chunk<T>(wv[j][r], xf[m][j], xb[m][j], s);
        acc[m][r] = s;
      }
    const int64_t cur_t = t;
    int64_t cur_rows[R];
    bool cur_ok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      cur_rows[r] = rows[r];
      cur_ok[r] = rok[r];
    }
    t += tstride;
    if (t0 + tstride < ntup) {
      set_rows(t);
      load_w();
    }

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
            for (int k = 1; k < KSPLIT; ++k) s += red[wave + k][m * R + r];
            acc[m][r] = s;
          }
      }
      __syncthreads();
    }

    if (kw != 0 || cur_t >= ntup) continue;
    if constexpr (EPI == EPI_ARGMAX) {
      T* logits = (T*)a.st->args.logits;
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        if (m < M) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if (cur_ok[r]) {
              const float v = round_to<T>(acc[m][r]);
              if (logits != nullptr && lane == m * R + r) store_f32<T>(logits, m * a.N + cur_rows[r], v);
              if (argmax_better(v, cur_rows[r], bv[m], bi[m])) {
                bv[m] = v;
                bi[m] = cur_rows[r];
              }
            }
          }
        }
      }
    } else if (em < M) {
      float va = 0.f, vb = 0.f;
#pragma unroll
      for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int p = 0; p < P; ++p)
          if (m == em && p == ep) {
            va = acc[m][p];
            vb = acc[m][P + p];
          }
      if (cur_t != (int64_t)blockIdx.x * SLOTS + slot) load_side<T, EPI, PP>(a, em, ep, cur_rows, cur_ok, pos, side);
      finish_pair<T, EPI>(a, em, cur_rows[ep], cur_rows[P + ep], cur_ok[ep], cur_ok[P + ep], va, vb, side, pos);
    }
  }
  if constexpr (EPI == EPI_ARGMAX) argmax_finish<MM, SLOTS>(a, M, slot, kw, bv, bi, best_v, best_i);
}

// ---------------------------------------------------------------------------
// gemv_lds_kernel: the input rows staged in LDS (any K that fits), for rows
// longer than the register path serves.
template <typename T, int MM, int KSPLIT, int PRO, int EPI>
__global__ __launch_bounds__(256) void gemv_lds_kernel(GemvArgs a) {
  extern __shared__ float xs[];  // [MM][K]
  __shared__ float red[4][MM * R];
  __shared__ float nrm[4][MM];
  __shared__ float best_v[4][MM];
  __shared__ int64_t best_i[4][MM];

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
        T* logits = (T*)a.st->args.logits;
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
                const int head = (int)row_a / D;
                const int i = (int)row_a % D;
                const int b = m / s.T, tt = m % s.T;
                if (head < s.Hq + s.Hkv) {
                  // rotate(x) = x * cos + rotate_half(x) * sin, fp32, each op
                  // rounded, then cast (rope.py:61-62)
                  const int64_t pos = st->args.positions[tt];
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
                  } else if (!st->halted) {
                    const int64_t g = head - s.Hq;
                    T* kc = (T*)st->args.k_cache + (int64_t)a.layer * s.B * s.Hkv * s.S * D;
                    const int64_t base = (((int64_t)b * s.Hkv + g) * s.S + st->args.cache_len + tt) * D;
                    store_f32<T>(kc, base + i, oa);
                    store_f32<T>(kc, base + i + half, ob);
                  }
                } else if (!st->halted) {
                  const int64_t g = head - s.Hq - s.Hkv;
                  T* vc = (T*)st->args.v_cache + (int64_t)a.layer * s.B * s.Hkv * s.S * D;
                  const int64_t base = (((int64_t)b * s.Hkv + g) * s.S + st->args.cache_len + tt) * D;
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

  if constexpr (EPI == EPI_ARGMAX) argmax_finish<MM, SLOTS>(a, M, slot, kw, bv, bi, best_v, best_i);
}


// ---------------------------------------------------------------------------
// gemv_split_kernel: M <= 4 rows with K split over blocks (no RMSNorm
// prologue; plain, residual and SwiGLU epilogues). The grid is tuples x
// segments: block b takes segment b % nseg (seg_bytes of every row) of tuple
// b / nseg, so a long-K matrix is spread over many more blocks than it has
// tuples and every block issues all of its loads at once (JMAX 16-byte
// chunks per row per lane, input chunks beside them, no LDS stage). Each
// block reduces its segment to one fp32 partial per (row, tuple row) and
// stores it at device scope; one lane then counts the block in on the
// tuple's arrival word (agent-scope acq_rel add). The block that arrives
// last adds the nseg partials in segment order, the same sum whatever the
// arrival order, runs the epilogue and puts the word back to 0 for the next
// launch. No block ever waits for another.
template <typename T, int MM, int JMAX, int EPI>
__global__ __launch_bounds__(256) void gemv_split_kernel(GemvArgs a, int nseg, uint32_t seg_bytes) {
  constexpr int V = Vec<T>::N;
  __shared__ float red[4][MM * R];
  __shared__ int last;
  const int tid = threadIdx.x, lane = tid & 63, kw = tid >> 6;
  const int M = (int)a.M;
  const int64_t t = blockIdx.x / nseg;
  const int seg = (int)(blockIdx.x % nseg);
  const uint32_t row_bytes = (uint32_t)(a.K * (int64_t)sizeof(T));
  const uint32_t seg0 = (uint32_t)seg * seg_bytes;
  const uint32_t len = min(seg_bytes, row_bytes - seg0);

  int64_t ra = 0, rb = 0;
  tuple_rows<EPI>(t, a, ra, rb);
  int64_t rows[R];
  bool rok[R];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    rows[p] = ra + p;
    rows[P + p] = rb + p;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) rok[r] = row_valid<EPI>(rows[r], a);

  // lane l of wave kw reads chunks kw * 64 + l + 256 j of the segment; past
  // its end (or the row's) the buffer loads return zeros
  uint32_t coff[JMAX];
#pragma unroll
  for (int j = 0; j < JMAX; ++j) coff[j] = (uint32_t)((kw * 64 + lane + j * 256) * 16);
  uint4 wv[JMAX][R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const __amdgpu_buffer_rsrc_t rs =
        span_rsrc((const char*)a.w + (rok[r] ? rows[r] : 0) * (int64_t)row_bytes + seg0, rok[r] ? len : 0u);
#pragma unroll
    for (int j = 0; j < JMAX; ++j) wv[j][r] = span_load16<W_AUX>(rs, coff[j]);
  }
  uint4 xb[MM][JMAX];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    const __amdgpu_buffer_rsrc_t xr =
        span_rsrc((const char*)a.x + (m < M ? m : 0) * a.ldx * (int64_t)sizeof(T) + seg0, m < M ? len : 0u);
#pragma unroll
    for (int j = 0; j < JMAX; ++j) xb[m][j] = span_load16<0>(xr, coff[j]);
  }
  // the epilogue's side inputs, loaded now (by the lanes of wave 0 that may
  // finish a pair), not after the last block has seen every count
  const int em = lane / P, ep = lane % P;
  float side[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (kw == 0 && em < M) load_side<T, EPI>(a, em, ep, rows, rok, 0, side);

  float acc[MM][R];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    float xf[JMAX][V];
#pragma unroll
    for (int j = 0; j < JMAX; ++j) unpack16(xb[m][j], xf[j], (T*)nullptr);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < JMAX; ++j) s = dot_chunk<T>(wv[j][r], xf[j], xb[m][j], s);
      acc[m][r] = wave_sum(s);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r) red[kw][m * R + r] = acc[m][r];
  }
  __syncthreads();
  // wave 0 publishes the block's partials, then counts the block in
  float* part = a.split_part + (t * nseg + seg) * (MM * R);
  if (kw == 0) {
    if (lane < MM * R) {
      const float v = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
      __hip_atomic_store(part + lane, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // The partials are device-coherent stores (sc1); the wave waits for
    // their completion (vmcnt(0)) before it counts the block in. This is
    // what an agent-scope release does for atomic stores, without its L2
    // write-back, which covers the whole cache and costs far more than the
    // GEMV. The builtin's operand encodes vmcnt(0) expcnt(7) lgkmcnt(15).
    __builtin_amdgcn_s_waitcnt(0x0F70);
    if (lane == 0) {
      const uint32_t old = __hip_atomic_fetch_add(a.split_count + t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = old == (uint32_t)(nseg - 1);
      if (last) __hip_atomic_store(a.split_count + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if (!last || kw != 0) return;

  // ---- the last block: segment sums in order, then the epilogue -----------
  // (device-coherent loads, issued after every count was seen)
  if (em >= M) return;
  const float* tp = a.split_part + t * nseg * (MM * R);
  float va = 0.f, vb = 0.f;
  for (int s = 0; s < nseg; ++s) {
    va += __hip_atomic_load(tp + s * (MM * R) + em * R + ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    vb += __hip_atomic_load(tp + s * (MM * R) + em * R + P + ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  finish_pair<T, EPI>(a, em, rows[ep], rows[P + ep], rok[ep], rok[P + ep], va, vb, side, 0);
}

// ---------------------------------------------------------------------------
// Decode rows 5..32 (bf16) on MFMA. The same tuples and epilogues as the
// register GEMV, with 16 weight rows per tuple: rows ra + 0..7 and rb + 0..7
// (pairs (ra + p, rb + p): SwiGLU gate j / up I + j, RoPE dims i / i + D/2,
// plain rows t*16 + p / t*16 + 8 + p). A wave owns one tuple and a K range
// (KSPLIT waves share a tuple and add their sums in a fixed order), and runs
// v_mfma_f32_16x16x32_bf16 with the input rows as the A operand (rows 0-15 and
// 16-31: two fragments; lane l reads x[l % 16][8 (l / 16) + 0..7] straight
// from memory) and the weights as B (lane l reads 16 bytes of tuple row
// l % 16). Lane l's accumulator r is then (row 4 (l / 16) + r, tuple row
// l % 16), so the pair partner of a result sits in lane l ^ 8. The RMSNorm
// prologue computes each input row's scale from the block's K-split partial
// sums and normalizes the A fragments in registers (layer.py:39-42).
constexpr int P16 = 8;  // pairs per 16-row tuple

template <int EPI>
__device__ __forceinline__ void tuple16_rows(int64_t t, const GemvArgs& a, int64_t& ra, int64_t& rb) {
  if constexpr (EPI == EPI_SWIGLU) {
    ra = t * P16;
    rb = a.N + t * P16;
  } else if constexpr (is_qkv<EPI>()) {
    const int half = a.a.D / 2;
    const int per_head = half / P16;
    const int t32 = (int)t;  // 32-bit division
    ra = (int64_t)(t32 / per_head) * a.a.D + (t32 % per_head) * P16;
    rb = ra + half;
  } else {
    ra = t * 2 * P16;
    rb = ra + P16;
  }
}

template <int EPI>
__host__ __device__ __forceinline__ int64_t num_tuples16(const GemvArgs& a) {
  if constexpr (EPI == EPI_SWIGLU) return a.N / P16;
  if constexpr (is_qkv<EPI>()) return (int64_t)(a.a.Hq + 2 * a.a.Hkv) * (a.a.D / 2) / P16;
  return cdiv(a.N, 2 * P16);
}

typedef __bf16 bf16x8_m __attribute__((ext_vector_type(8)));
typedef float f32x4_m __attribute__((ext_vector_type(4)));

// One k step's A fragments normalized in registers: o = dtype((x * r) * w).
__device__ __forceinline__ uint4 norm_chunk(const uint4& xb, const uint4& wb, float r) {
  float xf[8], wf[8], o[8];
  unpack16(xb, xf, (bf16*)nullptr);
  unpack16(wb, wf, (bf16*)nullptr);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = mul_rn(mul_rn(xf[e], r), wf[e]);
  return pack_bf16x8(o);
}

// Single-batch staging: a wave's K range is at most MF_ONE steps, i.e. 32
// 16-byte chunks per row. Rows are loaded coalesced (lane l takes chunk
// l % 32 of row l / 32 + 2 t: 512 contiguous bytes per row instead of the
// operand layout's 64) and stored to wave-private LDS with chunk c of row r
// at slot c ^ (r & 15), so the 16 lanes that read one operand column (16
// rows, one chunk) hit 16 different bank groups. The weights pass first,
// then the input rows, through the same 16 KiB per wave (two blocks per CU
// stay resident).
constexpr int MF_STAGE_CH = 32;
constexpr int MF_X_STAGE = 32 * MF_STAGE_CH * 16;   // the 32 input rows of a wave's K range
constexpr int MF_W_STAGE = 16 * MF_STAGE_CH * 16;   // one tuple's 16 weight rows
__device__ __forceinline__ uint32_t mf_slot(int r, int c) { return (uint32_t)((r * MF_STAGE_CH + (c ^ (r & 15))) * 16); }
template <int NT>
constexpr int mf_wave_stage() { return MF_X_STAGE > NT * MF_W_STAGE ? MF_X_STAGE : NT * MF_W_STAGE; }
template <int NT>
constexpr int mf_stage_bytes() { return 4 * mf_wave_stage<NT>(); }

template <int PRO, int EPI, int KSPLIT, int NT, int NB, bool MULTI, bool HV = false>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(GemvArgs a) {
  // A wave owns NT tuples that share each A fragment it loads, over a K
  // range of steps of 32. !MULTI: the range fits one batch of NB steps and
  // every load (weights, input rows, norm weight) goes out at once, so the
  // kernel waits one memory round trip; the RMSNorm scale comes from the
  // same input registers. MULTI: batches of NB steps, each batch's loads
  // issued while the previous one is multiplied (no norm prologue).
  // HV (half rows): a block takes one 16-row half of the input rows (one A
  // fragment: half the input loads, norm work and MFMAs); blocks b and b + 8,
  // on one XCD, share a tuple, so its weights come from that XCD's L2 the
  // second time.
  constexpr int SLOTS = 4 / KSPLIT;
  constexpr int WAUX = HV ? 0 : AUX_NT;  // weight-load policy (more than 16 rows: plain)
  constexpr int NF = HV ? 1 : 2;  // A fragments (16-row halves) a block multiplies
  constexpr uint32_t OOBW = 0xffffffffu;
  static_assert(!(MULTI && PRO == PRO_NORM), "the norm prologue needs the K range in one batch");
  __shared__ float nrm[4][32];
  __shared__ f32x4_m red[4][NT][2][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kw = wave % KSPLIT, slot = wave / KSPLIT;
  const int M = (int)a.M;
  const int64_t K = a.K;
  const int half = HV ? (int)((blockIdx.x >> 3) & 1) : 0;
  const int64_t tblk = HV ? ((int64_t)(blockIdx.x >> 4) << 3) | (blockIdx.x & 7) : (int64_t)blockIdx.x;
  const int64_t t0 = (tblk * SLOTS + slot) * NT;
  auto frow = [&](int f) { return HV ? 16 * half : 16 * f; };  // first input row of fragment f
  const int64_t ntup = num_tuples16<EPI>(a);
  const int nidx = lane & 15, kq = lane >> 4;
  const int64_t w_rows = EPI == EPI_SWIGLU ? 2 * a.N : a.N;
  // whole-matrix resources; lane offsets past a row's K or past M read zeros
  const __amdgpu_buffer_rsrc_t wr = span_rsrc(a.w, (uint32_t)(w_rows * K * 2));
  const __amdgpu_buffer_rsrc_t xr = span_rsrc(a.x, (uint32_t)(((int64_t)(M - 1) * a.ldx + K) * 2));
  const __amdgpu_buffer_rsrc_t nr = span_rsrc(a.norm_w, PRO == PRO_NORM ? (uint32_t)(K * 2) : 0u);
  int64_t ra[NT], rb[NT];
  uint32_t wbase[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const bool live = t0 + j < ntup;
    ra[j] = rb[j] = 0;
    if (live) tuple16_rows<EPI>(t0 + j, a, ra[j], rb[j]);
    const int64_t wrow = nidx < P16 ? ra[j] + nidx : rb[j] + (nidx - P16);
    wbase[j] = live && row_valid<EPI>(wrow, a) ? (uint32_t)(wrow * K * 2) : OOBW;
  }
  const int m0 = frow(0) + nidx, m1 = 16 + nidx;
  const uint32_t xb0 = m0 < M ? (uint32_t)((int64_t)m0 * a.ldx * 2) : OOBW;
  const uint32_t xb1 = !HV && m1 < M ? (uint32_t)((int64_t)m1 * a.ldx * 2) : OOBW;
  const int64_t nsteps = cdiv(K, 32), per = cdiv(nsteps, KSPLIT);
  const int64_t s_begin = kw * per, s_end = std::min(nsteps, s_begin + per);
  auto off = [&](uint32_t base, int64_t s) -> uint32_t {
    const int64_t k = s * 32 + kq * 8;
    return (base != OOBW && s < s_end && k < K) ? base + (uint32_t)(k * 2) : OOBW;
  };
  struct Batch {
    uint4 w[NB][NT], xa[NB], xc[NB], nw[NB];
  };
  auto issue = [&](Batch& b, int64_t s0) {
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) b.w[i][j] = span_load16<WAUX>(wr, off(wbase[j], s0 + i));
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      b.xa[i] = span_load16<0>(xr, off(xb0, s0 + i));
      if constexpr (!HV) b.xc[i] = span_load16<0>(xr, off(xb1, s0 + i));
      if constexpr (PRO == PRO_NORM) b.nw[i] = span_load16<0>(nr, off(0u, s0 + i));
    }
  };
  f32x4_m acc[NT][2];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) acc[j][h] = f32x4_m{0.f, 0.f, 0.f, 0.f};
  auto consume = [&](Batch& b) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const bf16x8_m aa = __builtin_bit_cast(bf16x8_m, b.xa[i]);
      const bf16x8_m ac = __builtin_bit_cast(bf16x8_m, HV ? b.xa[i] : b.xc[i]);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const bf16x8_m bw = __builtin_bit_cast(bf16x8_m, b.w[i][j]);
        acc[j][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aa, bw, acc[j][0], 0, 0, 0);
        if constexpr (!HV) acc[j][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ac, bw, acc[j][1], 0, 0, 0);
      }
    }
  };

  Batch b0;
  // !MULTI: the wave's whole K range staged through LDS (coalesced loads)
  extern __shared__ __attribute__((aligned(16))) char mf_stage[];
  char* xs_lds = mf_stage + wave * mf_wave_stage<NT>();
  char* ws_lds = xs_lds;
  uint4 wl[NT][8], xl[16];
  const int64_t kb = s_begin * 32;
  const int nch = (int)std::max<int64_t>(0, std::min<int64_t>((s_end - s_begin) * 4, (K - kb) / 8));
  if constexpr (!MULTI) {
    // input rows first (the norm prologue needs them first), then weights
#pragma unroll
    for (int t = 0; t < 8 * NF; ++t) {
      const int q = lane + 64 * (t + 8 * half), r = q >> 5, c = q & 31;  // rows frow(0) ..
      const bool ok = r < M && c < nch;
      xl[t] = span_load16<0>(xr, ok ? (uint32_t)(((int64_t)r * a.ldx + kb + 8 * c) * 2) : OOBW);
    }
    if constexpr (PRO == PRO_NORM) {
#pragma unroll
      for (int i = 0; i < NB; ++i) b0.nw[i] = span_load16<0>(nr, off(0u, s_begin + i));
    }
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int q = lane + 64 * t, r = q >> 5, c = q & 31;
        const int64_t wrow = r < P16 ? ra[j] + r : rb[j] + (r - P16);
        const bool ok = t0 + j < ntup && row_valid<EPI>(wrow, a) && c < nch;
        wl[j][t] = span_load16<WAUX>(wr, ok ? (uint32_t)((wrow * K + kb + 8 * c) * 2) : OOBW);
      }
  } else {
    issue(b0, s_begin);
  }
  // the epilogue's side inputs (residual, QKV bias, the single-token RoPE
  // rows) load now, underneath the weights, not after the products: lane
  // l < 8 of a K-split leader finishes pair l of each tuple for rows
  // 4 (l / 16) + r and 16 + 4 (l / 16) + r
  constexpr int NSIDE = EPI == EPI_RESID ? 16 : (EPI == EPI_QKV_ROPE1 ? 6 : (EPI == EPI_QKV_ROPE ? 2 : 1));
  float sv[NT][NSIDE];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int p = nidx & (P16 - 1);
    const int64_t row_a = ra[j] + p, row_b = rb[j] + p;
    const bool oka = t0 + j < ntup && row_valid<EPI>(row_a, a), okb = t0 + j < ntup && row_valid<EPI>(row_b, a);
#pragma unroll
    for (int q = 0; q < NSIDE; ++q) sv[j][q] = 0.f;
    if constexpr (EPI == EPI_RESID) {
      const bf16* aux = (const bf16*)a.aux;
#pragma unroll
      for (int h = 0; h < NF; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = frow(h) + 4 * kq + r;
          const int mm = m < M ? m : 0;
          sv[j][h * 8 + r] = load_f32<bf16>(aux, mm * a.ldy + (oka ? row_a : 0));
          sv[j][h * 8 + 4 + r] = load_f32<bf16>(aux, mm * a.ldy + (okb ? row_b : 0));
        }
    } else if constexpr (is_qkv<EPI>()) {
      sv[j][0] = load_f32<bf16>((const bf16*)a.bias, oka ? row_a : 0);
      sv[j][1] = load_f32<bf16>((const bf16*)a.bias, okb ? row_b : 0);
      if constexpr (EPI == EPI_QKV_ROPE1) {
        const int D = a.a.D, i = (int)row_a % D;
        sv[j][2] = a.st->rope_cos[i];
        sv[j][3] = a.st->rope_sin[i];
        sv[j][4] = a.st->rope_cos[i + D / 2];
        sv[j][5] = a.st->rope_sin[i + D / 2];
      }
    }
  }
  if constexpr (!MULTI) {
    // coalesced rows -> swizzled LDS -> operand fragments: the input rows,
    // then (same wave-private buffer) the weights
    auto wave_sync = []() {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
#pragma unroll
    for (int t = 0; t < 8 * NF; ++t) {
      const int q = lane + 64 * (t + 8 * half);
      *(uint4*)(xs_lds + mf_slot(q >> 5, q & 31)) = xl[t];
    }
    wave_sync();
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      b0.xa[i] = *(const uint4*)(xs_lds + mf_slot(m0, 4 * i + kq));
      if constexpr (!HV) b0.xc[i] = *(const uint4*)(xs_lds + mf_slot(m1, 4 * i + kq));
    }
    wave_sync();
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int q = lane + 64 * t;
        *(uint4*)(ws_lds + j * MF_W_STAGE + mf_slot(q >> 5, q & 31)) = wl[j][t];
      }
    wave_sync();
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) b0.w[i][j] = *(const uint4*)(ws_lds + j * MF_W_STAGE + mf_slot(nidx, 4 * i + kq));
    if constexpr (PRO == PRO_NORM) {
      // sums of squares of this wave's K range (packed dots: exact products,
      // fp32 sums), over the four lanes of a row (l, l + 16, l + 32, l + 48),
      // then over the block's K-split waves in order
      float ss0 = 0.f, ss1 = 0.f;
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        ss0 = dot_chunk<bf16>(b0.xa[i], nullptr, b0.xa[i], ss0);
        if constexpr (!HV) ss1 = dot_chunk<bf16>(b0.xc[i], nullptr, b0.xc[i], ss1);
      }
      ss0 += __shfl_xor(ss0, 16);
      ss0 += __shfl_xor(ss0, 32);
      if constexpr (!HV) {
        ss1 += __shfl_xor(ss1, 16);
        ss1 += __shfl_xor(ss1, 32);
      }
      if (kq == 0) {
        nrm[wave][m0] = ss0;
        if constexpr (!HV) nrm[wave][m1] = ss1;
      }
      __syncthreads();
      float u0 = 0.f, u1 = 0.f;
      for (int k = 0; k < KSPLIT; ++k) {
        u0 += nrm[slot * KSPLIT + k][m0];
        if constexpr (!HV) u1 += nrm[slot * KSPLIT + k][m1];
      }
      const float r0 = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(u0, (float)K), a.eps)));
      const float r1 = HV ? 0.f : __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(u1, (float)K), a.eps)));
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        b0.xa[i] = norm_chunk(b0.xa[i], b0.nw[i], r0);
        if constexpr (!HV) b0.xc[i] = norm_chunk(b0.xc[i], b0.nw[i], r1);
      }
    }
    consume(b0);
  } else {
    Batch b1;
    for (int64_t s0 = s_begin; s0 < s_end; s0 += 2 * NB) {
      issue(b1, s0 + NB);
      consume(b0);
      if (s0 + 2 * NB < s_end) issue(b0, s0 + 2 * NB);
      consume(b1);
    }
  }

  if constexpr (KSPLIT > 1) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      red[wave][j][0][lane] = acc[j][0];
      if constexpr (!HV) red[wave][j][1][lane] = acc[j][1];
    }
    __syncthreads();
    // every wave adds the K-split tiles in wave order (the same sums in
    // every wave) and finishes accumulator register r = kw of each tile, so
    // the epilogue's work is spread over the block
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int h = 0; h < NF; ++h) {
        f32x4_m v = red[slot * KSPLIT][j][h][lane];
        for (int k = 1; k < KSPLIT; ++k) v += red[slot * KSPLIT + k][j][h][lane];
        acc[j][h] = v;
      }
  }
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    float pa0[4], pa1[4];  // the pair partners' sums (lane l ^ 8)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pa0[r] = __shfl_xor(acc[j][0][r], 8);
      pa1[r] = HV ? 0.f : __shfl_xor(acc[j][1][r], 8);
    }
    if (t0 + j >= ntup || nidx >= P16) continue;
    const int p = nidx;
    const int64_t row_a = ra[j] + p, row_b = rb[j] + p;
    const bool oka = row_valid<EPI>(row_a, a), okb = row_valid<EPI>(row_b, a);
    float side[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if constexpr (is_qkv<EPI>()) {
      side[4] = sv[j][0];
      side[5] = sv[j][1];
    }
    if constexpr (EPI == EPI_QKV_ROPE1) {
      side[0] = sv[j][2];
      side[1] = sv[j][3];
      side[2] = sv[j][4];
      side[3] = sv[j][5];
    }
#pragma unroll
    for (int h = 0; h < NF; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (KSPLIT > 1 && r % KSPLIT != kw) continue;
        const int m = frow(h) + 4 * kq + r;
        if (m >= M) continue;
        const float va = acc[j][h][r], vb = h ? pa1[r] : pa0[r];
        int64_t pos = 0;
        if constexpr (EPI == EPI_QKV_ROPE) {
          const int D = a.a.D, i = (int)row_a % D;
          pos = a.st->args.positions[m % a.a.T];
          if ((int)row_a / D < a.a.Hq + a.a.Hkv && pos >= 0 && pos < a.max_pos) {
            side[0] = a.cos_tab[pos * D + i];
            side[1] = a.sin_tab[pos * D + i];
            side[2] = a.cos_tab[pos * D + i + D / 2];
            side[3] = a.sin_tab[pos * D + i + D / 2];
          }
        } else if constexpr (EPI == EPI_RESID) {
          side[0] = sv[j][h * 8 + r];
          side[1] = sv[j][h * 8 + 4 + r];
        }
        finish_pair<bf16, EPI>(a, m, row_a, row_b, oka, okb, va, vb, side, pos);
      }
  }
}

// steps of 32 per wave that one batch holds (the whole K range of a wave
// when it fits: the norm prologue needs that)
constexpr int MF_ONE = 8;

// ---------------------------------------------------------------------------
// gemv_mfma_loop_kernel: the single-batch MFMA GEMV for products with many
// tuples (the batch-32 gate/up: 608, the LM head: 9,496). A block's input
// fragments, normalized once, serve several tuples in turn (t = blockIdx.x,
// + gridDim.x, ...): the RMSNorm prologue, about 650 of the 1,130 VALU
// instructions per wave when every tuple has a block of its own, is paid
// once per block. Each tuple's weights are staged like gemv_mfma_kernel's;
// the loads of the tuples MF_LOOP_PD on go out before the current tuple's
// products (register buffers in rotation), and the K-split partial tiles
// alternate between two LDS buffers, so a tuple costs one block barrier.
// The two buffers (8 KB each) sit in the second halves of waves 0 and 1's
// input stages, which the weight stages leave free: 64.5 KB of LDS a block,
// two blocks a CU.
#ifndef MINITP_MF_LOOP_PD
#define MINITP_MF_LOOP_PD 2
#endif
// weights through the wave's LDS stage (1) or loaded in the operand layout (0)
#ifndef MINITP_MF_LOOP_STAGE
#define MINITP_MF_LOOP_STAGE 1
#endif
template <int PRO, int EPI, int WAUX>
__global__ __launch_bounds__(256) void gemv_mfma_loop_kernel(GemvArgs a) {
  static_assert(EPI == EPI_STORE || EPI == EPI_SWIGLU, "the tuple loop serves the store and SwiGLU epilogues");
  constexpr int MF_LOOP_PD = MINITP_MF_LOOP_PD;  // tuples whose weight loads are in flight
  constexpr int NB = 8;  // steps of 32 per wave (the single-batch form)
  constexpr uint32_t OOBW = 0xffffffffu;
  static_assert(4 * 2 * 64 * (int)sizeof(f32x4_m) == MF_W_STAGE && 2 * MF_W_STAGE == MF_X_STAGE, "LDS plan");
  __shared__ float nrm[4][32];
  extern __shared__ __attribute__((aligned(16))) char mf_stage[];
  const int tid = threadIdx.x, lane = tid & 63, kw = tid >> 6;
  const int M = (int)a.M;
  const int64_t K = a.K;
  const int64_t ntup = num_tuples16<EPI>(a);
  const int nidx = lane & 15, kq = lane >> 4;
  const int64_t w_rows = EPI == EPI_SWIGLU ? 2 * a.N : a.N;
  const __amdgpu_buffer_rsrc_t wr = span_rsrc(a.w, (uint32_t)(w_rows * K * 2));
  const __amdgpu_buffer_rsrc_t xr = span_rsrc(a.x, (uint32_t)(((int64_t)(M - 1) * a.ldx + K) * 2));
  const __amdgpu_buffer_rsrc_t nr = span_rsrc(a.norm_w, PRO == PRO_NORM ? (uint32_t)(K * 2) : 0u);
  const int m0 = nidx, m1 = 16 + nidx;
  const int64_t nsteps = cdiv(K, 32), per = cdiv(nsteps, 4);
  const int64_t s_begin = kw * per, s_end = std::min(nsteps, s_begin + per);
  const int64_t kb = s_begin * 32;
  const int nch = (int)std::max<int64_t>(0, std::min<int64_t>((s_end - s_begin) * 4, (K - kb) / 8));
  char* st_lds = mf_stage + kw * MF_X_STAGE;
  auto wave_sync = []() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // staged weight loads: lane l, load u takes chunk l % 32 of tuple row
  // l / 32 + 2 u (rows 0..7: ra + r, 8..15: rb + r - 8)
  const uint32_t wstep = (uint32_t)((EPI == EPI_SWIGLU ? P16 : 2 * P16) * K * 2);
  uint32_t wbase[8];
  bool wok[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int q = lane + 64 * u, r = q >> 5, c = q & 31;
    const int64_t row0 = r < P16 ? r : (EPI == EPI_SWIGLU ? a.N : P16) + (r - P16);
    wbase[u] = (uint32_t)((row0 * K + kb + 8 * c) * 2);
    wok[u] = c < nch;
  }
  auto load_w = [&](int64_t t, uint4 (&wl)[8]) {
    int64_t ra = 0, rb = 0;
    const bool live = t < ntup;
#if !MINITP_MF_LOOP_STAGE
    if (live) tuple16_rows<EPI>(t, a, ra, rb);
#endif
#if MINITP_MF_LOOP_STAGE
    // tuple t's rows are tuple 0's moved by t x (rows a tuple) x K: the
    // offsets are a per-lane base plus one uniform step. Prefetches past the
    // last tuple read zeros (their SwiGLU gate rows would land on up rows).
    // In the last tuple, rows past the product read zeros (past the buffer's
    // end) or, for SwiGLU gate rows past N, up rows whose outputs are never
    // stored.
    (void)ra;
    (void)rb;
    const uint32_t tof = (uint32_t)t * wstep;
#pragma unroll
    for (int u = 0; u < 8; ++u) wl[u] = span_load16<WAUX>(wr, live && wok[u] ? wbase[u] + tof : OOBW);
#else
    // straight into the operand layout: row nidx, chunk 4 i + kq
    const int64_t wrow = nidx < P16 ? ra + nidx : rb + (nidx - P16);
    const bool rok = live && row_valid<EPI>(wrow, a);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int c = 4 * i + kq;
      wl[i] = span_load16<WAUX>(wr, rok && c < nch ? (uint32_t)((wrow * K + kb + 8 * c) * 2) : OOBW);
    }
#endif
  };

  // ---- input rows (and norm weight), then the first tuple's weights -------
  uint4 xl[16], nw[NB], wl[MF_LOOP_PD][8];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int q = lane + 64 * u, r = q >> 5, c = q & 31;
    const bool ok = r < M && c < nch;
    xl[u] = span_load16<0>(xr, ok ? (uint32_t)(((int64_t)r * a.ldx + kb + 8 * c) * 2) : OOBW);
  }
  if constexpr (PRO == PRO_NORM) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int64_t s = s_begin + i, k = s * 32 + kq * 8;
      nw[i] = span_load16<0>(nr, s < s_end && k < K ? (uint32_t)(k * 2) : OOBW);
    }
  }
#pragma unroll
  for (int j = 0; j < MF_LOOP_PD; ++j) load_w(blockIdx.x + j * (int64_t)gridDim.x, wl[j]);
  // Keep the scheduler from moving the input rows' LDS writes, and the waits
  // for those rows, above the weight loads.
  __builtin_amdgcn_sched_barrier(0);

  // ---- A fragments through the wave's LDS stage, normalized once ----------
  uint4 xa[NB], xc[NB];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int q = lane + 64 * u;
    *(uint4*)(st_lds + mf_slot(q >> 5, q & 31)) = xl[u];
  }
  wave_sync();
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    xa[i] = *(const uint4*)(st_lds + mf_slot(m0, 4 * i + kq));
    xc[i] = *(const uint4*)(st_lds + mf_slot(m1, 4 * i + kq));
  }
  wave_sync();
  if constexpr (PRO == PRO_NORM) {
    float ss0 = 0.f, ss1 = 0.f;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      ss0 = dot_chunk<bf16>(xa[i], nullptr, xa[i], ss0);
      ss1 = dot_chunk<bf16>(xc[i], nullptr, xc[i], ss1);
    }
    ss0 += __shfl_xor(ss0, 16);
    ss0 += __shfl_xor(ss0, 32);
    ss1 += __shfl_xor(ss1, 16);
    ss1 += __shfl_xor(ss1, 32);
    if (kq == 0) {
      nrm[kw][m0] = ss0;
      nrm[kw][m1] = ss1;
    }
    __syncthreads();  // also: every wave is done with its input stage
    float u0 = 0.f, u1 = 0.f;
    for (int k = 0; k < 4; ++k) {
      u0 += nrm[k][m0];
      u1 += nrm[k][m1];
    }
    const float r0 = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(u0, (float)K), a.eps)));
    const float r1 = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(u1, (float)K), a.eps)));
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      xa[i] = norm_chunk(xa[i], nw[i], r0);
      xc[i] = norm_chunk(xc[i], nw[i], r1);
    }
  } else {
    __syncthreads();  // every wave is done with its input stage (the sum buffers overlay them)
  }

  // ---- tuples ---------------------------------------------------------------
  // Outputs go out through a buffer resource, every lane issuing the same
  // stores each tuple (an offset past the end drops one): with no store
  // behind a branch, the compiler's count of memory operations in flight
  // stays exact across the loop, and the wait before a tuple's weights are
  // staged lets the loads of the tuples after it stay in flight.
  bf16* yp = (bf16*)(a.y != nullptr ? a.y : a.st->args.logits);
  const __amdgpu_buffer_rsrc_t yr = span_rsrc(yp, (uint32_t)(((int64_t)(M - 1) * a.ldy + a.N) * 2));
  const __amdgpu_buffer_rsrc_t br = span_rsrc(a.bias, a.bias != nullptr ? (uint32_t)(a.N * 2) : 0u);
  const int kwu = __builtin_amdgcn_readfirstlane(kw);
  auto tuple = [&](const int64_t t, const int it, uint4 (&wl)[8]) {
    int64_t ra = 0, rb = 0;
    tuple16_rows<EPI>(t, a, ra, rb);
    // SwiGLU: lane nidx < 8 finishes gate row ra + nidx with its up partner
    // (lane nidx + 8); plain store: every lane finishes its own column
    const int p = nidx & (P16 - 1);
    const int64_t row_a = EPI == EPI_STORE ? (nidx < P16 ? ra + p : rb + p) : ra + p;
    const bool oka = (EPI == EPI_STORE || nidx < P16) && row_valid<EPI>(row_a, a);
    float bias_a = 0.f;
    if constexpr (EPI == EPI_STORE)  // a zero-length resource reads zeros
      bias_a = bf16_to_f32((uint16_t)__builtin_amdgcn_raw_buffer_load_b16(br, oka ? (uint32_t)(row_a * 2) : OOBW, 0, 0));
    // this tuple's weights -> fragments; those MF_LOOP_PD tuples on go out
    uint4 w[NB];
#if MINITP_MF_LOOP_STAGE
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int q = lane + 64 * u;
      *(uint4*)(st_lds + mf_slot(q >> 5, q & 31)) = wl[u];
    }
    wave_sync();
#pragma unroll
    for (int i = 0; i < NB; ++i) w[i] = *(const uint4*)(st_lds + mf_slot(nidx, 4 * i + kq));
    wave_sync();
#else
#pragma unroll
    for (int i = 0; i < NB; ++i) w[i] = wl[i];
#endif
    load_w(t + MF_LOOP_PD * (int64_t)gridDim.x, wl);
    f32x4_m acc[2] = {f32x4_m{0.f, 0.f, 0.f, 0.f}, f32x4_m{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const bf16x8_m bw = __builtin_bit_cast(bf16x8_m, w[i]);
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_m, xa[i]), bw, acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_m, xc[i]), bw, acc[1], 0, 0, 0);
    }
    // K-split sum (two alternating buffers: one barrier per tuple): every
    // wave the same sums in wave order, wave kw finishing register kw
    // (planes [register][wave][h][lane]: a wave reads only its register's
    // plane, 2 KiB instead of 8, every read conflict-free)
    float* rb_buf = (float*)(mf_stage + (it & 1) * MF_X_STAGE + MF_W_STAGE);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) rb_buf[((r * 4 + kw) * 2 + h) * 64 + lane] = acc[h][r];
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      // register kw of the sum (row 16 h + 4 kq + kw, column nidx), and the
      // partner column nidx ^ 8 (row_ror:8 within each 16-lane row)
      const float* pl = rb_buf + (kwu * 4 * 2 + h) * 64 + lane;
      const float va = ((pl[0] + pl[2 * 64]) + pl[4 * 64]) + pl[6 * 64];
      const int m = h * 16 + 4 * kq + kwu;
      const bool okm = m < M;
      if constexpr (EPI == EPI_STORE) {
        const uint16_t ya = f32_to_bf16(va + bias_a);
        __builtin_amdgcn_raw_buffer_store_b16(ya, yr, okm && oka ? (uint32_t)((m * a.ldy + row_a) * 2) : OOBW, 0, 0);
      } else {
        const float vb = dpp_f32<0x128>(0.f, va);
        const uint16_t ya = f32_to_bf16(swiglu<bf16>(round_to<bf16>(va), round_to<bf16>(vb)));
        __builtin_amdgcn_raw_buffer_store_b16(ya, yr, okm && oka ? (uint32_t)((m * a.ldy + row_a) * 2) : OOBW, 0, 0);
      }
    }
  };
  int it = 0;
  for (int64_t tb = blockIdx.x; tb < ntup; tb += MF_LOOP_PD * (int64_t)gridDim.x) {
#pragma unroll
    for (int j = 0; j < MF_LOOP_PD; ++j) {
      const int64_t t = tb + j * (int64_t)gridDim.x;
      if (t >= ntup) break;
      tuple(t, it++, wl[j]);
    }
  }
}


// ---------------------------------------------------------------------------
// gemv_mfma_split_kernel: decode rows 5..32 (bf16) with K split over blocks
// as well as over a block's 4 waves, no RMSNorm prologue. The grid is groups
// of NT tuples (x) by K segments of seg_steps steps of 32 (y): the few-tuple
// products (QKV: 72 tuples at the 0.5B shape, o_proj 56, down 56) spread over
// hundreds of blocks, and each block loads only its segment of the input
// rows. Every block issues all of its loads at once (at most MF_ONE steps
// per wave), multiplies, adds its waves' tiles in order, and stores the
// block's 16 x 32 tile per tuple device-coherent; the block that brings the
// group's arrival word to nseg adds the segments in order and runs the
// epilogue (the same sum whatever the arrival order), then puts the word
// back to 0. Each extra device-scope round trip (partial stores, the
// count, the partial loads) costs about as much as the load phase, so this
// pays only where the unsplit form leaves most of the chip idle for long:
// the down projection at the 0.5B shape (K = 4,864, 56 tuples).
constexpr int AUX_SC1 = 16;  // buffer-op cache policy: device scope (sc1)

__device__ __forceinline__ void store16_dev(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4_m v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, AUX_SC1);
}
__device__ __forceinline__ f32x4_m load16_dev(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4_m, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX_SC1));
}

template <int EPI, int NT>
__global__ __launch_bounds__(256) void gemv_mfma_split_kernel(GemvArgs a, int nseg, int seg_steps) {
  constexpr uint32_t OOBW = 0xffffffffu;
  __shared__ f32x4_m red[4][NT][2][64];
  __shared__ int last;
  const int tid = threadIdx.x, lane = tid & 63, kw = tid >> 6;
  const int M = (int)a.M;
  const int64_t K = a.K;
  const int64_t grp = blockIdx.x;
  const int seg = (int)blockIdx.y;
  const int64_t t0 = grp * NT;
  const int64_t ntup = num_tuples16<EPI>(a);
  const int nidx = lane & 15, kq = lane >> 4;
  const int64_t w_rows = EPI == EPI_SWIGLU ? 2 * a.N : a.N;
  const __amdgpu_buffer_rsrc_t wr = span_rsrc(a.w, (uint32_t)(w_rows * K * 2));
  const __amdgpu_buffer_rsrc_t xr = span_rsrc(a.x, (uint32_t)(((int64_t)(M - 1) * a.ldx + K) * 2));
  int64_t ra[NT], rb[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    ra[j] = rb[j] = 0;
    if (t0 + j < ntup) tuple16_rows<EPI>(t0 + j, a, ra[j], rb[j]);
  }
  const int m0 = nidx, m1 = 16 + nidx;
  const int64_t nsteps = cdiv(K, 32);
  const int64_t sb = (int64_t)seg * seg_steps, se = std::min(nsteps, sb + seg_steps);
  const int64_t per = cdiv((int64_t)seg_steps, 4);
  const int64_t s_begin = sb + kw * per, s_end = std::min(se, s_begin + per);
  // the wave's K range staged through LDS as in gemv_mfma_kernel:
  // coalesced loads (input rows first), swizzled wave-private tiles
  extern __shared__ __attribute__((aligned(16))) char mf_stage[];
  char* st_lds = mf_stage + kw * mf_wave_stage<NT>();
  const int64_t kb = s_begin * 32;
  const int nch = (int)std::max<int64_t>(0, std::min<int64_t>((s_end - s_begin) * 4, (K - kb) / 8));
  uint4 wl[NT][8], xl[16];
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const int q = lane + 64 * t, r = q >> 5, c = q & 31;
    const bool ok = r < M && c < nch;
    xl[t] = span_load16<0>(xr, ok ? (uint32_t)(((int64_t)r * a.ldx + kb + 8 * c) * 2) : OOBW);
  }
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int q = lane + 64 * t, r = q >> 5, c = q & 31;
      const int64_t wrow = r < P16 ? ra[j] + r : rb[j] + (r - P16);
      const bool ok = t0 + j < ntup && row_valid<EPI>(wrow, a) && c < nch;
      wl[j][t] = span_load16<AUX_NT>(wr, ok ? (uint32_t)((wrow * K + kb + 8 * c) * 2) : OOBW);
    }
  // the epilogue's side inputs, loaded underneath the weights (only the
  // block that finishes a group uses them)
  constexpr int NSIDE = EPI == EPI_RESID ? 16 : (EPI == EPI_QKV_ROPE1 ? 6 : (EPI == EPI_QKV_ROPE ? 2 : 1));
  float sv[NT][NSIDE];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int p = nidx & (P16 - 1);
    const int64_t row_a = ra[j] + p, row_b = rb[j] + p;
    const bool oka = t0 + j < ntup && row_valid<EPI>(row_a, a), okb = t0 + j < ntup && row_valid<EPI>(row_b, a);
#pragma unroll
    for (int q = 0; q < NSIDE; ++q) sv[j][q] = 0.f;
    if constexpr (EPI == EPI_RESID) {
      const bf16* aux = (const bf16*)a.aux;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = h * 16 + 4 * kq + r;
          const int mm = m < M ? m : 0;
          sv[j][h * 8 + r] = load_f32<bf16>(aux, mm * a.ldy + (oka ? row_a : 0));
          sv[j][h * 8 + 4 + r] = load_f32<bf16>(aux, mm * a.ldy + (okb ? row_b : 0));
        }
    } else if constexpr (is_qkv<EPI>()) {
      sv[j][0] = load_f32<bf16>((const bf16*)a.bias, oka ? row_a : 0);
      sv[j][1] = load_f32<bf16>((const bf16*)a.bias, okb ? row_b : 0);
      if constexpr (EPI == EPI_QKV_ROPE1) {
        const int D = a.a.D, i = (int)row_a % D;
        sv[j][2] = a.st->rope_cos[i];
        sv[j][3] = a.st->rope_sin[i];
        sv[j][4] = a.st->rope_cos[i + D / 2];
        sv[j][5] = a.st->rope_sin[i + D / 2];
      }
    }
  }
  uint4 w[MF_ONE][NT], xa[MF_ONE], xc[MF_ONE];
  {
    auto wave_sync = []() {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int q = lane + 64 * t;
      *(uint4*)(st_lds + mf_slot(q >> 5, q & 31)) = xl[t];
    }
    wave_sync();
#pragma unroll
    for (int i = 0; i < MF_ONE; ++i) {
      xa[i] = *(const uint4*)(st_lds + mf_slot(m0, 4 * i + kq));
      xc[i] = *(const uint4*)(st_lds + mf_slot(m1, 4 * i + kq));
    }
    wave_sync();
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int q = lane + 64 * t;
        *(uint4*)(st_lds + j * MF_W_STAGE + mf_slot(q >> 5, q & 31)) = wl[j][t];
      }
    wave_sync();
#pragma unroll
    for (int i = 0; i < MF_ONE; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) w[i][j] = *(const uint4*)(st_lds + j * MF_W_STAGE + mf_slot(nidx, 4 * i + kq));
  }
  f32x4_m acc[NT][2];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) acc[j][h] = f32x4_m{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < MF_ONE; ++i) {
    const bf16x8_m aa = __builtin_bit_cast(bf16x8_m, xa[i]), ac = __builtin_bit_cast(bf16x8_m, xc[i]);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const bf16x8_m bw = __builtin_bit_cast(bf16x8_m, w[i][j]);
      acc[j][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aa, bw, acc[j][0], 0, 0, 0);
      acc[j][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ac, bw, acc[j][1], 0, 0, 0);
    }
  }
  // the block's tile: its waves' K ranges added in order
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    red[kw][j][0][lane] = acc[j][0];
    red[kw][j][1][lane] = acc[j][1];
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t pr = span_rsrc(a.split_part, (uint32_t)a.split_part_bytes);
  auto part_off = [&](int64_t sg, int j, int h) -> uint32_t {
    return (uint32_t)(((((grp * nseg + sg) * NT + j) * 2 + h) * 64 + lane) * 16);
  };
  if (kw == 0) {
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f32x4_m v = red[0][j][h][lane];
        for (int k = 1; k < 4; ++k) v += red[k][j][h][lane];
        store16_dev(pr, part_off(seg, j, h), v);
      }
    // device-coherent stores complete (vmcnt(0) expcnt(7) lgkmcnt(15))
    // before the block is counted in: an agent-scope release without its
    // whole-L2 write-back
    __builtin_amdgcn_s_waitcnt(0x0F70);
    if (lane == 0) {
      const uint32_t old = __hip_atomic_fetch_add(a.split_count + grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = old == (uint32_t)(nseg - 1);
      if (last) __hip_atomic_store(a.split_count + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if (!last) return;
  {
    // ---- the group's last block: segments in order (every wave the same
    // sums), then the epilogue, accumulator register r = kw per wave ----
    // (SB segments' loads in flight at a time; past nseg they read zeros)
    constexpr int SB = 8 / NT;
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) acc[j][h] = f32x4_m{0.f, 0.f, 0.f, 0.f};
    for (int sg0 = 0; sg0 < nseg; sg0 += SB) {
      f32x4_m v[SB][NT][2];
#pragma unroll
      for (int u = 0; u < SB; ++u)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int h = 0; h < 2; ++h) v[u][j][h] = load16_dev(pr, sg0 + u < nseg ? part_off(sg0 + u, j, h) : OOBW);
#pragma unroll
      for (int u = 0; u < SB; ++u)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int h = 0; h < 2; ++h) acc[j][h] += v[u][j][h];
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      float pa0[4], pa1[4];  // the pair partners' sums (lane l ^ 8)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pa0[r] = __shfl_xor(acc[j][0][r], 8);
        pa1[r] = __shfl_xor(acc[j][1][r], 8);
      }
      if (t0 + j >= ntup || nidx >= P16) continue;
      const int p = nidx;
      const int64_t row_a = ra[j] + p, row_b = rb[j] + p;
      const bool oka = row_valid<EPI>(row_a, a), okb = row_valid<EPI>(row_b, a);
      float side[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if constexpr (is_qkv<EPI>()) {
        side[4] = sv[j][0];
        side[5] = sv[j][1];
      }
      if constexpr (EPI == EPI_QKV_ROPE1) {
        side[0] = sv[j][2];
        side[1] = sv[j][3];
        side[2] = sv[j][4];
        side[3] = sv[j][5];
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (r != kw) continue;
          const int m = h * 16 + 4 * kq + r;
          if (m >= M) continue;
          const float va = acc[j][h][r], vb = h ? pa1[r] : pa0[r];
          int64_t pos = 0;
          if constexpr (EPI == EPI_QKV_ROPE) {
            const int D = a.a.D, i = (int)row_a % D;
            pos = a.st->args.positions[m % a.a.T];
            if ((int)row_a / D < a.a.Hq + a.a.Hkv && pos >= 0 && pos < a.max_pos) {
              side[0] = a.cos_tab[pos * D + i];
              side[1] = a.sin_tab[pos * D + i];
              side[2] = a.cos_tab[pos * D + i + D / 2];
              side[3] = a.sin_tab[pos * D + i + D / 2];
            }
          } else if constexpr (EPI == EPI_RESID) {
            side[0] = sv[j][h * 8 + r];
            side[1] = sv[j][h * 8 + 4 + r];
          }
          finish_pair<bf16, EPI>(a, m, row_a, row_b, oka, okb, va, vb, side, pos);
        }
    }
  }
}

// Split form geometry: NT tuples per group, nseg segments of seg_steps.
struct MfSplit {
  int nt, nseg, seg_steps;
  int64_t groups, part_bytes;
};
// Blocks the split aims at (segments = this / groups, rounded up). At the
// 0.5B batch-32 down projection (56 groups, 152 steps of 32), one box, two
// runs each: 5 segments 1.0523-1.0535 ms a step, 6 1.0416-1.0418, 7
// 1.0417-1.0434, 8 1.0479-1.0488.
#ifndef MINITP_MF_TARGET_BLOCKS
#define MINITP_MF_TARGET_BLOCKS 320
#endif
#ifndef MINITP_MF_MIN_STEPS
#define MINITP_MF_MIN_STEPS 1
#endif
template <int EPI>
MfSplit mf_split(const GemvArgs& a) {
  MfSplit g{};
  const int64_t ntup = num_tuples16<EPI>(a), nsteps = cdiv(a.K, 32);
  g.nt = ntup >= 512 ? 2 : 1;
  g.groups = cdiv(ntup, g.nt);
  const int64_t lo = cdiv(nsteps, 4 * MF_ONE);
  const int64_t hi = std::max<int64_t>(1, nsteps / (4 * MINITP_MF_MIN_STEPS));
  int64_t n = std::max(lo, std::min(cdiv((int64_t)MINITP_MF_TARGET_BLOCKS, g.groups), hi));
  g.seg_steps = (int)cdiv(nsteps, n);
  g.nseg = (int)cdiv(nsteps, (int64_t)g.seg_steps);
  g.part_bytes = g.groups * g.nseg * g.nt * 2 * 64 * 16;
  return g;
}

template <int EPI>
bool mf_split_ok(const GemvArgs& a) {
  if constexpr (!(EPI == EPI_STORE || EPI == EPI_RESID || EPI == EPI_SWIGLU || is_qkv<EPI>())) {
    return false;
  } else {
    if (a.split_part == nullptr || a.split_count == nullptr) return false;
    const MfSplit g = mf_split<EPI>(a);
    return g.groups <= SPLIT_MAX_TUPLES && g.part_bytes <= a.split_part_bytes &&
           a.split_part_bytes < (1LL << 32) && (int64_t)g.seg_steps <= 4 * MF_ONE;
  }
}

template <int EPI, int NT>
int launch_mfma_split_nt(hipStream_t st, const GemvArgs& a, const MfSplit& g) {
  const dim3 grid((unsigned)g.groups, (unsigned)g.nseg);
  auto kern = gemv_mfma_split_kernel<EPI, NT>;
  const int lds = mf_stage_bytes<NT>();
  const int rc = ensure_lds_limit((const void*)kern, lds);
  if (rc) return rc;
  hipLaunchKernelGGL(kern, grid, dim3(256), lds, st, a, g.nseg, g.seg_steps);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

template <int EPI>
int launch_mfma_split(hipStream_t st, const GemvArgs& a) {
  if constexpr (!(EPI == EPI_STORE || EPI == EPI_RESID || EPI == EPI_SWIGLU || is_qkv<EPI>())) {
    set_error("gemv: no split form for epilogue %d", EPI);
    return MINITP_ERR_UNSUPPORTED;
  } else {
    const MfSplit g = mf_split<EPI>(a);
    return g.nt == 2 ? launch_mfma_split_nt<EPI, 2>(st, a, g) : launch_mfma_split_nt<EPI, 1>(st, a, g);
  }
}

// The tuple-loop form from MINITP_MF_LOOP_MIN tuples: at least
// MINITP_MF_LOOP_PER tuples a block, and at most MINITP_MF_LOOP_BLOCKS blocks
// (two a CU). Measured on the batch-32 decode (kernel trace): gate/up (608
// tuples) 10.3 us at 2 a block, 8.9-9.3 at 3, 9.9 at 4; the LM head (9,496
// tuples) 56 us on 500 blocks, 60 on 256, 100 on 128. Two tuples' loads in
// flight against one: LM head 56 against 59 us, gate/up within noise; three:
// slower (1.167 against 1.143 ms a step).
#ifndef MINITP_MF_LOOP_MIN
#define MINITP_MF_LOOP_MIN 512
#endif
#ifndef MINITP_MF_LOOP_PER
#define MINITP_MF_LOOP_PER 3
#endif
#ifndef MINITP_MF_LOOP_BLOCKS
#define MINITP_MF_LOOP_BLOCKS 512
#endif
// Above 16 input rows the one-tuple MFMA form runs each 16-row half in a
// block of its own (HV): half the input loads, RMSNorm work and MFMAs per
// block on twice the blocks. 0.5B batch 32 (QKV 72 tuples, o_proj 56):
// 1.123-1.125 -> 1.067-1.068 ms a step.
#ifndef MINITP_MF_HALVES
#define MINITP_MF_HALVES 1
#endif
template <int PRO, int EPI, int NT>
int launch_mfma_nt(hipStream_t st, const GemvArgs& a, int64_t ntup) {
  const unsigned grid = (unsigned)cdiv(ntup, NT);
  const int64_t per_wave = cdiv(cdiv(a.K, 32), 4);
  if constexpr (EPI == EPI_STORE || EPI == EPI_SWIGLU) {
    // (32-bit weight offsets: at most 1 GiB of weights)
    const int64_t w_bytes = (EPI == EPI_SWIGLU ? 2 : 1) * a.N * a.K * 2;
    if (per_wave <= MF_ONE && NT == 1 && ntup >= MINITP_MF_LOOP_MIN && w_bytes < (1LL << 30)) {
      // many tuples: several a block, the input rows' prologue shared
      // (weights plain above 16 rows for the gate/up; the LM head's 272 MB
      // stream stays non-temporal: 53 against 58 us at batch 32, kernel trace)
      auto kern = a.M > MINITP_MF_PLAIN_ROWS && EPI == EPI_SWIGLU ? gemv_mfma_loop_kernel<PRO, EPI, 0>
                                                                  : gemv_mfma_loop_kernel<PRO, EPI, AUX_NT>;
      const int lds = 4 * MF_X_STAGE;
      const int rc = ensure_lds_limit((const void*)kern, lds);
      if (rc) return rc;
      const int64_t per = std::max<int64_t>(MINITP_MF_LOOP_PER, cdiv(ntup, (int64_t)MINITP_MF_LOOP_BLOCKS));
      hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(ntup, per)), dim3(256), lds, st, a);
      MINITP_LAUNCH_CHECK();
      return MINITP_OK;
    }
  }
  if (per_wave <= MF_ONE) {
    const int lds = mf_stage_bytes<NT>();
    if (NT == 1 && a.M > 16 && MINITP_MF_HALVES) {
      // each 16-row half of the input rows in a block of its own
      auto kern = gemv_mfma_kernel<PRO, EPI, 4, NT, MF_ONE, false, true>;
      const int rc = ensure_lds_limit((const void*)kern, lds);
      if (rc) return rc;
      hipLaunchKernelGGL(kern, dim3((unsigned)(cdiv(ntup, (int64_t)8) * 16)), dim3(256), lds, st, a);
    } else {
      auto kern = gemv_mfma_kernel<PRO, EPI, 4, NT, MF_ONE, false>;
      const int rc = ensure_lds_limit((const void*)kern, lds);
      if (rc) return rc;
      hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, st, a);
    }
  } else if constexpr (PRO == PRO_NORM) {
    set_error("gemv: the RMSNorm prologue on MFMA serves K <= %d", 4 * 32 * MF_ONE);
    return MINITP_ERR_UNSUPPORTED;
  } else {
    hipLaunchKernelGGL((gemv_mfma_kernel<PRO, EPI, 4, NT, 4, true>), dim3(grid), dim3(256), 0, st, a);
  }
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

template <int PRO, int EPI>
int launch_mfma(hipStream_t st, const GemvArgs& a) {
  if constexpr (EPI == EPI_ARGMAX) {
    set_error("gemv: the argmax epilogue serves at most 4 rows");
    return MINITP_ERR_UNSUPPORTED;
  } else {
    // with split buffers and no norm prologue: K split over blocks too
    if constexpr (PRO == PRO_NONE) {
      if (mf_split_ok<EPI>(a)) return launch_mfma_split<EPI>(st, a);
    }
    // K split over the block's 4 waves, one tuple per block (two per block
    // measured slower at every shape once the loads were staged: 13.0
    // against 12.2 us for the batch-32 gate/up)
    const int64_t ntup = num_tuples16<EPI>(a);
    return launch_mfma_nt<PRO, EPI, 1>(st, a, ntup);
  }
}

template <typename T, int MM, int KSPLIT, int JMAX, int PRO, int EPI, int PP>
int launch_reg_pp(hipStream_t st, const GemvArgs& a) {
  const int64_t slots = 4 / KSPLIT;
  const int64_t cap = EPI == EPI_ARGMAX ? gemv_argmax_partials(a.N) : a.max_grid > 0 ? a.max_grid : MAX_GRID;
  const int grid = (int)std::min<int64_t>(cdiv(num_tuples<EPI, PP>(a), slots), cap);
  hipLaunchKernelGGL((gemv_reg_kernel<T, MM, KSPLIT, JMAX, PRO, EPI, PP>), dim3(grid), dim3(256), 0, st, a);
  MINITP_LAUNCH_CHECK();
  if constexpr (EPI == EPI_ARGMAX) {
    return launch_argmax_merge(st, a.part_val, a.part_idx, grid, a.M, nullptr, 0, a.st);
  }
  return MINITP_OK;
}

// Tuples of one pair (two rows, twice the blocks) where tuples of P pairs
// would leave CUs without a block: at the 0.5B decode shape QKV 72 -> 144
// blocks (3.42 -> 3.26 us) and down 224 -> 448 (4.15 -> 3.95 us); the
// larger launches (gate/up 7.01 -> 7.52 us, the LM head 42.6 -> 43.1 us)
// keep P pairs. The same per-row sums either way, so the results are the
// same bit for bit.
template <typename T, int MM, int KSPLIT, int JMAX, int PRO, int EPI>
int launch_reg(hipStream_t st, const GemvArgs& a) {
  if constexpr (EPI != EPI_ARGMAX && PRO != PRO_PART_NORM) {
    if (cdiv(num_tuples<EPI>(a), (int64_t)(4 / KSPLIT)) < device_cus())
      return launch_reg_pp<T, MM, KSPLIT, JMAX, PRO, EPI, 1>(st, a);
  }
  return launch_reg_pp<T, MM, KSPLIT, JMAX, PRO, EPI, P>(st, a);
}

template <typename T, int MM, int PRO, int EPI>
int launch_lds(hipStream_t st, const GemvArgs& a) {
  auto kern = gemv_lds_kernel<T, MM, 4, PRO, EPI>;
  const int lds = (int)(MM * a.K * sizeof(float));
  int rc = ensure_lds_limit((const void*)kern, lds);
  if (rc) return rc;
  const int64_t cap = EPI == EPI_ARGMAX ? gemv_argmax_partials(a.N) : MAX_GRID;
  const int grid = (int)std::min<int64_t>(num_tuples<EPI>(a), cap);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, st, a);
  MINITP_LAUNCH_CHECK();
  if constexpr (EPI == EPI_ARGMAX) {
    return launch_argmax_merge(st, a.part_val, a.part_idx, grid, a.M, nullptr, 0, a.st);
  }
  return MINITP_OK;
}

template <typename T, int MM, int JMAX, int EPI>
int launch_split_j(hipStream_t st, const GemvArgs& a, int nseg, int64_t seg_chunks) {
  const int64_t grid = num_tuples<EPI>(a) * nseg;
  hipLaunchKernelGGL((gemv_split_kernel<T, MM, JMAX, EPI>), dim3((unsigned)grid), dim3(256), 0, st, a, nseg,
                     (uint32_t)(seg_chunks * 16));
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

// Segments of at most 256 x SPLIT_JMAX chunks, sized evenly.
template <typename T, int MM, int EPI>
int launch_split(hipStream_t st, const GemvArgs& a) {
  const int64_t nchunk = a.K / Vec<T>::N;
  const int nseg = (int)cdiv(nchunk, 256 * SPLIT_JMAX);
  const int64_t seg_chunks = cdiv(nchunk, nseg);
  if ((nseg - 1) * seg_chunks >= nchunk || nseg > SPLIT_MAX_SEG || num_tuples<EPI>(a) > SPLIT_MAX_TUPLES) {
    set_error("gemv split: %lld chunks in %d segments of %lld", (long long)nchunk, nseg, (long long)seg_chunks);
    return MINITP_ERR_UNSUPPORTED;
  }
  switch (cdiv(seg_chunks, 256)) {
    case 1:
      return launch_split_j<T, MM, 1, EPI>(st, a, nseg, seg_chunks);
    case 2:
      return launch_split_j<T, MM, 2, EPI>(st, a, nseg, seg_chunks);
    case 3:
      return launch_split_j<T, MM, 3, EPI>(st, a, nseg, seg_chunks);
    default:
      return launch_split_j<T, MM, 4, EPI>(st, a, nseg, seg_chunks);
  }
}

// The split form serves rows of more than SPLIT_MIN_CHUNKS chunks when the
// caller gave it its buffers, the input is not normalized in the prologue
// and the tuples and segments fit them.
template <typename T, int PRO, int EPI>
bool use_split(const GemvArgs& a) {
  if constexpr (PRO != PRO_NONE || !(EPI == EPI_STORE || EPI == EPI_RESID || EPI == EPI_SWIGLU)) {
    return false;
  } else {
    const int64_t nchunk = a.K / Vec<T>::N;
    return a.split_part != nullptr && a.split_count != nullptr && nchunk > SPLIT_MIN_CHUNKS &&
           a.split_part_bytes >= gemv_split_part_bytes(1) &&
           num_tuples<EPI>(a) <= SPLIT_MAX_TUPLES && cdiv(nchunk, 256 * SPLIT_JMAX) <= SPLIT_MAX_SEG &&
           a.K * (int64_t)sizeof(T) < (1LL << 31);
  }
}

template <typename T, int MM, int PRO, int EPI>
int pick_k(hipStream_t st, const GemvArgs& a) {
  const int64_t nchunk = a.K / Vec<T>::N;
  if constexpr (MM == 1 && PRO == PRO_NONE && (EPI == EPI_STORE || EPI == EPI_RESID || EPI == EPI_SWIGLU))
    if (use_split<T, PRO, EPI>(a)) return launch_split<T, MM, EPI>(st, a);
  if (nchunk <= 128) return launch_reg<T, MM, 1, 2, PRO, EPI>(st, a);
  if constexpr (MM <= 2) {
    // up to 512 chunks: bf16 rows split K over four waves, one tuple a block
    // (at the 7B decode the 1,152 QKV and 896 o_proj tuples then spread over
    // twice the blocks: 365.5 -> 370.5 tok/s; gate/up the same either way);
    // fp32 rows over two waves, two tuples a block
    if (nchunk <= 512) {
      if constexpr (sizeof(T) == 2) return launch_reg<T, MM, 4, 2, PRO, EPI>(st, a);
      return launch_reg<T, MM, 2, 4, PRO, EPI>(st, a);
    }
    if (nchunk <= REG_MAX_CHUNKS) return launch_reg<T, MM, 4, 4, PRO, EPI>(st, a);
  }
  if constexpr (MM == 1) return launch_lds<T, MM, PRO, EPI == EPI_QKV_ROPE1 ? EPI_QKV_ROPE : EPI>(st, a);
  set_error("gemv: M=%lld with K=%lld is served by the GEMM path", (long long)a.M, (long long)a.K);
  return MINITP_ERR_UNSUPPORTED;
}

template <typename T, int PRO, int EPI>
int pick_m(hipStream_t st, const GemvArgs& a) {
  if constexpr (sizeof(T) == 2) {
    if (a.M >= MF_MIN_ROWS) return launch_mfma<PRO, EPI>(st, a);
  }
  if (a.M == 1) return pick_k<T, 1, PRO, EPI>(st, a);
  if (a.M == 2) return pick_k<T, 2, PRO, EPI>(st, a);
  return pick_k<T, 4, PRO, EPI>(st, a);
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
      return a.a.T == 1 ? pick_m<T, PRO, EPI_QKV_ROPE1>(st, a) : pick_m<T, PRO, EPI_QKV_ROPE>(st, a);
    case EPI_ARGMAX:
      return pick_m<T, PRO, EPI_ARGMAX>(st, a);
  }
  set_error("gemv: unknown epilogue %d", epi);
  return MINITP_ERR_ARG;
}

template <typename T>
int launch_part_swiglu_t(hipStream_t st, const GemvArgs& a) {
  const int64_t nchunk = a.K / Vec<T>::N;
  // (K <= PART_MAX_K: bf16 rows are at most 128 chunks, fp32 rows 256)
  if (nchunk <= 128) return launch_reg<T, 1, 1, 2, PRO_PART_NORM, EPI_SWIGLU>(st, a);
  if constexpr (sizeof(T) == 4) return launch_reg<T, 1, 2, 4, PRO_PART_NORM, EPI_SWIGLU>(st, a);
  set_error("gemv: partial-sum prologue row of %lld chunks", (long long)nchunk);
  return MINITP_ERR_UNSUPPORTED;
}

}  // namespace

bool gemv_part_supported(int dtype, int64_t K, int nparts) {
  const int v = dtype == MINITP_F32 ? 4 : 8;
  return nparts >= 1 && nparts <= PART_MAX_PARTS && K >= v && K % v == 0 && K <= PART_MAX_K;
}

// Compute units of the current device (cached per device).
static int device_cus() {
  static std::mutex mu;
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cus[dev] == 0) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cus[dev];
}

int launch_gemv_part_swiglu(hipStream_t st, int dtype, const GemvArgs& a_in) {
  if (a_in.M != 1 || !gemv_part_supported(dtype, a_in.K, a_in.nparts) || a_in.part == nullptr ||
      a_in.x_out == nullptr) {
    set_error("gemv: partial-sum prologue needs one row, K <= %lld, 1..%d partial rows (M=%lld K=%lld parts=%d)",
              (long long)PART_MAX_K, PART_MAX_PARTS, (long long)a_in.M, (long long)a_in.K, a_in.nparts);
    return MINITP_ERR_UNSUPPORTED;
  }
  // One block per CU: every block reads all the partial rows once, so fewer
  // blocks read less (0.5B decode: 608 blocks 0.553 ms a token, 256 blocks
  // 0.517, 320 0.543).
  GemvArgs a = a_in;
  if (a.max_grid <= 0) a.max_grid = device_cus();
  return dtype == MINITP_F32 ? launch_part_swiglu_t<float>(st, a) : launch_part_swiglu_t<bf16>(st, a);
}

int64_t gemv_split_part_bytes(int64_t M) {
  const int64_t reg = (int64_t)SPLIT_MAX_TUPLES * SPLIT_MAX_SEG * 4 * R * sizeof(float);
  return M >= MF_MIN_ROWS && M <= 32 ? std::max<int64_t>(reg, 16LL << 20) : reg;
}

// Block count (and so partial count per row) of the LM-head argmax GEMV.
int64_t gemv_argmax_partials(int64_t N) { return std::min<int64_t>(cdiv(cdiv(N, R), 4), 1024); }

// The register path keeps the input rows in registers (M * JMAX chunks per
// lane): M <= 4 up to 128 chunks per row, M <= 2 up to 1024; M == 1 beyond
// that stages the input in LDS (up to 80 KiB). Other shapes run the GEMM.
bool gemv_supported(int dtype, int64_t M, int64_t K) {
  const int v = dtype == MINITP_F32 ? 4 : 8;
  // bf16 rows MF_MIN_ROWS..32 run the MFMA form (K a multiple of 8, rows under 2 GiB)
  if (gemv_mfma_rows(dtype, M)) return K % v == 0 && K * 2 < (1LL << 31);
  if (M < 1 || M > 4 || K % v != 0) return false;
  const int64_t nchunk = K / v;
  if (nchunk <= 128) return true;
  if (nchunk <= REG_MAX_CHUNKS) return M <= 2;
  return M == 1 && K * 4 <= 80 * 1024;
}

// The RMSNorm prologue holds a wave's whole K range: on the MFMA form that
// is K <= 4 waves x 8 steps x 32.
bool gemv_norm_supported(int dtype, int64_t M, int64_t K) {
  if (!gemv_supported(dtype, M, K)) return false;
  return !gemv_mfma_rows(dtype, M) || K <= 4 * 32 * MF_ONE;
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
