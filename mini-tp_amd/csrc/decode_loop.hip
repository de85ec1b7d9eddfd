// Persistent single-token decode: one launch runs the whole batch-1 forward
// (TPQwen2ForCausalLM.forward, layer.py:91-124, at T == 1) and the greedy
// pick (generation.py:54-67), instead of one graph node per kernel.
//
// Why: a decode step at the 0.5B shape reads ~1 GB of weights in ~125 us at
// HBM speed, but as a graph of 122 dependent kernels every node costs a
// fixed ~5 us (dispatch, cache writeback / invalidate at each kernel
// boundary, ramp-up, drain). Here one block per CU stays resident for the
// whole step and blocks hand results to each other through "LL" words:
// 8-byte words holding a 32-bit payload and the 32-bit epoch of the step
// that wrote them, stored and loaded as relaxed agent-scope atomics. A
// consumer spins until every word it needs carries the current epoch, so a
// hand-off is one store plus one load through the device coherence point
// (~0.45 us within an XCD, ~0.65 us across), with no counters, fences or
// cache flushes. Every (layer, phase) has its own words, so no word is
// rewritten within a step; the epoch (kept in the workspace, bumped once per
// step) tells this step's words from the last.
//
// Four hand-offs per layer:
//   A  RMSNorm(x) -> QKV GEMV + bias -> RoPE -> q, k, v words; k, v also into
//      the KV cache (for later steps)                      [all blocks]
//   B  GQA attention of one KV group + that group's share of o_proj for a
//      slice of the output rows -> fp32 partial words      [Hkv x RS blocks]
//   C  x += dtype(sum of the group partials); RMSNorm -> gate/up GEMV ->
//      SwiGLU -> act words                                  [all blocks]
//   D  down GEMV -> dtype(down) words                       [all blocks]
// then RMSNorm -> LM head GEMV -> per-block argmax partial words, and block 0
// merges them into the token. Every block keeps its own copy of the residual
// stream x in LDS and applies both residual adds itself (layer.py:63-64), so
// x never travels.
//
// Roles inside a block (8 waves): wave 0 is the only wave that waits on
// hand-off words; it copies a phase's inputs into LDS and releases the block
// through s_barrier, and it issues every other small global load. Waves 1..7
// each stream the weights of ONE phase (the host splits them by bytes, e.g.
// 1 QKV, 1 o_proj, 3 gate/up, 2 down at the 0.5B shape): a wave consumes its
// phase's weights and at once issues the same phase's loads for the next
// layer, so weights are requested one layer before they are used and HBM
// latency stays off the critical path. Vector loads complete in issue order
// per wave; giving each wave a single stream is what keeps a wait for one
// load from also waiting for loads issued later (the compiler's waits are
// conservative across the layer loop), and it is why the waiting is left to
// wave 0 and why the barrier used here (s_barrier after the wave's own LDS
// traffic) never waits on global loads. The o_proj wave(s) also copy the K/V
// rows of the block's KV group global -> LDS (global_load_lds_dwordx4)
// during phase A, ahead of attention.
//
// Every wait is bounded by the wall clock: a wave that times out raises an
// abort word that ends every other wait, and sets an error bit the host
// reads back (minitp_qwen2_decode_check), so the grid always drains.
#include "common.h"
#include "decode_loop.h"
#include "kernels.h"

namespace minitp {

namespace {

constexpr int LT = LOOP_THREADS;
constexpr int LWAVES = LT / 64;
constexpr int NCW = LWAVES - 1;  // weight-streaming waves: 1 .. LWAVES - 1
constexpr int GMAXL = 8;         // query heads per KV group served
#ifndef LOOP_GATHER_INLINE
#define LOOP_GATHER_INLINE __forceinline__
#endif
// Register batches (chunk columns x rows) of each role's weight stream:
// everything a wave streams per layer at the 0.5B shape fits one batch;
// larger shapes run several batches per phase.
constexpr int JA = 2, SA = 8, JB = 2, SB = 8, JC = 2, SC = 14, JD = 10, SD = 2, JL = 2, SL = 14;  // J * S <= 28
constexpr int ATT_KV_BYTES = 64 * 1024;  // LDS for one K + V position tile

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ uint64_t ll_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_store(uint64_t* p, uint32_t epoch, uint32_t payload) {
  __hip_atomic_store(p, ((uint64_t)epoch << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Block barrier over LDS: this wave's LDS operations complete, then
// s_barrier. Outstanding global loads (prefetched weights) stay in flight.
__device__ __forceinline__ void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// Orders LDS traffic between the lanes of one wave.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename T>
struct Pk;  // LL packing: elements per word and per 16-byte chunk
template <>
struct Pk<bf16> {
  static constexpr int EPW = 2;
  static constexpr int VEC = 8;
};
template <>
struct Pk<float> {
  static constexpr int EPW = 1;
  static constexpr int VEC = 4;
};

// acc += <w, x> over one 16-byte chunk (same element type).
template <typename T>
__device__ __forceinline__ float dot16(const uint4& w, const uint4& x, float acc);
template <>
__device__ __forceinline__ float dot16<bf16>(const uint4& w, const uint4& x, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.x), __builtin_bit_cast(bf16x2_t, x.x), acc,
                                        false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.y), __builtin_bit_cast(bf16x2_t, x.y), acc,
                                        false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.z), __builtin_bit_cast(bf16x2_t, x.z), acc,
                                        false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.w), __builtin_bit_cast(bf16x2_t, x.w), acc,
                                         false);
}
template <>
__device__ __forceinline__ float dot16<float>(const uint4& w, const uint4& x, float acc) {
  acc = fmaf(__uint_as_float(w.x), __uint_as_float(x.x), acc);
  acc = fmaf(__uint_as_float(w.y), __uint_as_float(x.y), acc);
  acc = fmaf(__uint_as_float(w.z), __uint_as_float(x.z), acc);
  return fmaf(__uint_as_float(w.w), __uint_as_float(x.w), acc);
}

// Payload of one LL word from EPW consecutive output values (already
// rounded to T), and back.
template <typename T>
__device__ __forceinline__ uint32_t pack_word(const float* v);
template <>
__device__ __forceinline__ uint32_t pack_word<bf16>(const float* v) {
  return (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
}
template <>
__device__ __forceinline__ uint32_t pack_word<float>(const float* v) {
  return __float_as_uint(v[0]);
}
template <typename T>
__device__ __forceinline__ float word_elem(uint32_t w, int e);
template <>
__device__ __forceinline__ float word_elem<bf16>(uint32_t w, int e) {
  return __uint_as_float(e ? (w & 0xffff0000u) : (w << 16));
}
template <>
__device__ __forceinline__ float word_elem<float>(uint32_t w, int) {
  return __uint_as_float(w);
}

struct Ctx {
  const LoopParams* p;
  uint32_t epoch;
  int b, nb, tid, lane, wave, cw;  // cw: weight-wave index (wave - 1), -1 on wave 0
  // records the wall clock in the block's trace row (no-op when tracing is off)
  __device__ __forceinline__ void mark(int slot) const {
    if (p->trace && lane == 0) p->trace[((int64_t)b * p->trace_slots + slot) * LWAVES + wave] = wall_clock64();
  }
};

// Wave 0: copies hand-off words src[0..n) into raw[0..n) (LDS, 8 bytes
// each) and returns once every copied word carries the epoch. 16-byte pieces
// travel global -> LDS without registers, coherent at device scope (sc1, as
// the atomic loads); one wave-instruction moves 128 words, and only
// instructions still holding a word of an older epoch are repeated. On a
// timeout the wave raises the abort word; seeing the abort word ends the
// wait too. raw must have room for n rounded up to 128 words.
__device__ LOOP_GATHER_INLINE void ll_gather(const Ctx& c, const uint64_t* src, int n, uint64_t* raw) {
  const LoopParams& p = *c.p;
  const int nins = (n + 127) / 128;  // at most 64 (checked on the host)
  auto issue = [&](int j) {
    const int w = 2 * (j * 64 + c.lane);  // this lane's two words
    __builtin_amdgcn_global_load_lds((const void*)(src + (w < n ? w : 0)), (lds_void*)(raw + j * 128), 16, 0,
                                     16 /* sc1 */);
  };
  for (int j = 0; j < nins; ++j) issue(j);
  uint64_t pending = nins >= 64 ? ~0ull : (1ull << nins) - 1;
  const int64_t t0 = wall_clock64();
  for (int it = 1;; ++it) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    uint64_t still = 0;
    for (int j = 0; j < nins; ++j) {
      if (!((pending >> j) & 1)) continue;
      const int w = 2 * (j * 64 + c.lane);
      bool ok = true;
      if (w < n) ok = (uint32_t)(raw[w] >> 32) == c.epoch;
      if (w + 1 < n) ok = ok && (uint32_t)(raw[w + 1] >> 32) == c.epoch;
      if (!__all(ok)) still |= 1ull << j;
    }
    pending = still;
    if (!pending) break;
    if ((it & 15) == 0) {
      if (__hip_atomic_load(&p.ctrl[LOOP_CTRL_ABORT], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
      if (wall_clock64() - t0 > p.spin_limit) {
        if (c.lane == 0) {
          __hip_atomic_fetch_or(&p.ctrl[LOOP_CTRL_ERROR], (uint32_t)LOOP_ERR_TIMEOUT, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(&p.ctrl[LOOP_CTRL_ABORT], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        break;
      }
    }
    for (int j = 0; j < nins; ++j)
      if ((pending >> j) & 1) issue(j);
  }
}

__device__ __forceinline__ uint32_t payload(uint64_t w) { return (uint32_t)w; }

// A wave's rows of one weight matrix, read with buffer loads. Lane l owns
// the contiguous 16-byte chunks [l * cpl, l * cpl + cpl) of every row (nch
// chunks). The buffer resource covers the matrix from `base` (bytes bytes;
// the range check counts the scalar row offset too), and a chunk past the
// row end gets a lane offset beyond that range, so it reads as zeros. The
// wave has ns rows (slots); slot s starts at byte offset row_off(s).
struct Rows {
  const void* base;
  int bytes, ns, cpl, nch;
};

constexpr uint32_t OFF_RANGE = 0x80000000u;  // lane offset of a chunk past the row: reads zeros

__device__ __forceinline__ Rows make_rows(const void* base, int64_t bytes, int nch, int ns) {
  Rows q;
  q.base = base;
  q.bytes = (int)bytes;
  q.ns = ns;
  q.nch = nch;
  q.cpl = (nch + 63) / 64;
  return q;
}

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// A wave's register batch: BUFW 16-byte loads, used by each stream as
// J chunk columns x S slots (J * S <= BUFW), load (j, s) at index j * S + s.
constexpr int BUFW = 28;

// Issue the batch of slots [sb, sb + S) x columns [jb, jb + J). Every load
// is issued; loads outside the stream get an out-of-range lane offset and
// return zeros without touching memory, so the code has no branches.
// The buffer resource, built from wave-uniform values made explicitly
// uniform (otherwise the compiler may keep it in vector registers and wrap
// every load in a loop over distinct lane values).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const Rows& q) {
  const uint64_t a = (uint64_t)q.base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const int bytes = __builtin_amdgcn_readfirstlane(q.bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, bytes, 0x00020000);
}

template <int J, int S, class RowFn>
__device__ __forceinline__ void rows_issue(uint4 (&buf)[BUFW], const Rows& q, RowFn row_off, int sb, int jb,
                                           int lane) {
  static_assert(J * S <= BUFW, "batch larger than the register buffer");
  const __amdgpu_buffer_rsrc_t rsrc = rows_rsrc(q);
  uint32_t vo[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int cc = lane * q.cpl + jb + j;
    vo[j] = (cc < q.nch && jb + j < q.cpl) ? (uint32_t)cc * 16u : OFF_RANGE;
  }
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const bool live = sb + s < q.ns;
    const uint32_t so = live ? row_off(sb + s) : 0u;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const u32x4v v = __builtin_bit_cast(
          u32x4v, __builtin_amdgcn_raw_buffer_load_b128(rsrc, live ? vo[j] : OFF_RANGE,
                                                        __builtin_amdgcn_readfirstlane(so), 2 /* nt */));
      buf[j * S + s] = make_uint4(v.x, v.y, v.z, v.w);
    }
  }
}

// Dot every row of the stream with the LDS input x, batch by batch; the
// first batch (sb = 0, jb = 0) was issued by the caller. Hands each row's
// wave-reduced sum to done(slot, value) (executed by every lane).
template <typename T, int J, int S, class RowFn, class DoneFn>
__device__ __forceinline__ void rows_consume(uint4 (&buf)[BUFW], const Rows& q, RowFn row_off, const uint4* x,
                                             int lane, DoneFn done) {
  for (int sb = 0; sb < q.ns; sb += S) {
    float acc[S];
#pragma unroll
    for (int s = 0; s < S; ++s) acc[s] = 0.f;
    for (int jb = 0; jb < q.cpl; jb += J) {
      if (sb + jb > 0) rows_issue<J, S>(buf, q, row_off, sb, jb, lane);
      uint4 xj[J];
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int cc = lane * q.cpl + jb + j;
        xj[j] = (cc < q.nch && jb + j < q.cpl) ? x[cc] : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int j = 0; j < J; ++j) acc[s] = dot16<T>(buf[j * S + s], xj[j], acc[s]);
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const float v = wave_sum(acc[s]);
      if (sb + s < q.ns) done(sb + s, v);
    }
  }
}

// xin = dtype((x * rsqrt(mean(x^2) + eps)) * w), fp32 math (layer.py:39-42).
// w is the norm weight already copied into LDS (norm_fetch).
template <typename T>
__device__ __forceinline__ void block_rmsnorm(const Ctx& c, const float* xs, const T* w, T* xin, float* red) {
  const int H = c.p->H;
  float ss = 0.f;
  for (int i = c.tid; i < H; i += LT) ss = add_rn(ss, mul_rn(xs[i], xs[i]));
  ss = wave_sum(ss);
  if (c.lane == 0) red[c.wave] = ss;
  bar();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < LWAVES; ++k) tot += red[k];
  const float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(tot, (float)H), c.p->eps)));
  for (int i = c.tid; i < H; i += LT) store_f32<T>(xin, i, mul_rn(mul_rn(xs[i], r), load_f32<T>(w, i)));
  bar();
}

// Wave 0: copy `bytes` bytes of a global vector into LDS (1 KiB per
// wave-instruction; dst must have room for bytes rounded up to 1 KiB).
// Completion is awaited by the next ll_gather (or an explicit vmcnt wait).
__device__ __forceinline__ void lds_fetch(const Ctx& c, const void* src, int bytes, void* dst) {
  const char* s = (const char*)src;
  for (int j = 0; j * 1024 < bytes; ++j) {
    const int off = j * 1024 + c.lane * 16;
    __builtin_amdgcn_global_load_lds((const void*)(s + (off < bytes ? off : 0)), (lds_void*)((char*)dst + j * 1024), 16,
                                     0, 0);
  }
}

// Block-wide torch.argmax merge of (value, index) candidates held one per
// thread; the winner lands in sv[0] / si[0] (LDS), valid after the call.
__device__ __forceinline__ void block_argmax(const Ctx& c, float v, int64_t i, float* sv, int64_t* si) {
  wave_argmax(v, i);
  if (c.lane == 0) {
    sv[c.wave] = v;
    si[c.wave] = i;
  }
  bar();
  if (c.tid == 0) {
    for (int k = 1; k < LWAVES; ++k)
      if (argmax_better(sv[k], si[k], v, i)) {
        v = sv[k];
        i = si[k];
      }
    sv[0] = v;
    si[0] = i;
  }
  bar();
}

template <typename T, int D>
struct Loop {
  static constexpr int EPW = Pk<T>::EPW;
  static constexpr int VEC = Pk<T>::VEC;  // elements per 16-byte chunk
  static constexpr int HALF = D / 2;
  static constexpr int WPP = 2 / EPW;  // LL words per RoPE pair (a, b)
  static constexpr int PPR = D / VEC;  // 16-byte pieces per K / V row
  static constexpr int TP0 = ATT_KV_BYTES / 2 / (D * (int)sizeof(T));
  static constexpr int TP = TP0 > 256 ? 256 : TP0;  // positions per K / V tile
  static constexpr int LPR = D / 8;                  // P V lanes per value row (8 elements each)
  static constexpr int RPI = 64 / LPR;               // value rows per P V step

  // Hand-off word of RoPE pair (head hd, dim i): grouped by KV group, each
  // group's G q heads, then its k head, then its v head, so that a phase-B
  // block reads one contiguous range.
  __device__ __forceinline__ static int64_t qkv_word(const Ctx& c, int hd, int i) {
    const int Hq = c.p->Hq, Hkv = c.p->Hkv, G = c.p->G;
    int g, hh;
    if (hd < Hq) {
      g = hd / G;
      hh = hd % G;
    } else if (hd < Hq + Hkv) {
      g = hd - Hq;
      hh = G;
    } else {
      g = hd - Hq - Hkv;
      hh = G + 1;
    }
    return ((int64_t)(g * (G + 2) + hh) * HALF + i) * WPP;
  }

  // ---------------------------------------------------------------- phase A
  // Pair p = (head hd, dim i < D/2): rows hd * D + i and hd * D + i + D/2 of
  // the fused QKV weight (q heads, then k, then v; fused.py:60). Pair p goes
  // to block p % nb; local pair lp = p / nb to role wave lp % nrw, whose
  // slots 2t, 2t + 1 are the two rows of its t-th pair.
  __device__ __forceinline__ static int a_pairs_block(const Ctx& c) {
    const int npa = (c.p->Hq + 2 * c.p->Hkv) * HALF;
    return c.b < npa ? (npa - 1 - c.b) / c.nb + 1 : 0;
  }
  __device__ __forceinline__ static Rows a_q(const Ctx& c, const LoopLayerW& lw, int npb, int rw, int nrw) {
    const int my = rw < npb ? (npb - 1 - rw) / nrw + 1 : 0;
    return make_rows(lw.wqkv, (int64_t)(c.p->Hq + 2 * c.p->Hkv) * D * c.p->H * sizeof(T), c.p->H / VEC, 2 * my);
  }
  __device__ __forceinline__ static auto a_rows(const Ctx& c, int rw, int nrw) {
    const int nb = c.nb, b = c.b;
    const uint32_t row_bytes = (uint32_t)c.p->H * sizeof(T);
    return [=](int s) -> uint32_t {
      const int p = b + nb * (rw + nrw * (s >> 1));
      const int hd = p / HALF, i = p % HALF;
      return (uint32_t)(hd * D + i + (s & 1) * HALF) * row_bytes;
    };
  }

  // ---------------------------------------------------------------- phase B
  // Block b < Hkv * RS serves KV group g = b % Hkv and output rows
  // [r0, r1) = slice b / Hkv of RS equal slices of H; row r0 + k goes to
  // role wave k % nrw. The buffer starts at the group's first column of
  // o_proj, so a row is G * D long.
  __device__ __forceinline__ static void b_rows_range(const Ctx& c, int& g, int& r0, int& r1) {
    const int Hkv = c.p->Hkv, rs = c.nb / Hkv;
    g = c.b % Hkv;
    const int sl = c.b / Hkv;
    if (sl >= rs) {
      r0 = r1 = 0;
      return;
    }
    r0 = sl * c.p->H / rs;
    r1 = (sl + 1) * c.p->H / rs;
  }
  __device__ __forceinline__ static Rows b_q(const Ctx& c, const LoopLayerW& lw, int g, int nrows, int rw, int nrw) {
    const int my = rw < nrows ? (nrows - 1 - rw) / nrw + 1 : 0;
    const int64_t off = (int64_t)g * c.p->G * D;
    return make_rows((const T*)lw.wo + off, ((int64_t)c.p->H * c.p->Hq * D - off) * sizeof(T), c.p->G * D / VEC, my);
  }
  __device__ __forceinline__ static auto b_rows(const Ctx& c, int r0, int rw, int nrw) {
    const uint32_t row_bytes = (uint32_t)c.p->Hq * D * sizeof(T);
    return [=](int s) -> uint32_t { return (uint32_t)(r0 + rw + nrw * s) * row_bytes; };
  }

  // ---------------------------------------------------------------- phase C
  // Units of EPW intermediate indices; block b gets units [u0, u1). Block
  // row br: index j = u0 * EPW + br / 2, gate (br even) or up (odd) row;
  // block row br goes to role wave br % nrw.
  __device__ __forceinline__ static void c_range(const Ctx& c, int& u0, int& u1) {
    const int nu = c.p->I / EPW;
    u0 = c.b * nu / c.nb;
    u1 = (c.b + 1) * nu / c.nb;
  }
  __device__ __forceinline__ static Rows c_q(const Ctx& c, const LoopLayerW& lw, int nrows, int rw, int nrw) {
    const int my = rw < nrows ? (nrows - 1 - rw) / nrw + 1 : 0;
    return make_rows(lw.wgu, (int64_t)2 * c.p->I * c.p->H * sizeof(T), c.p->H / VEC, my);
  }
  __device__ __forceinline__ static auto c_rows(const Ctx& c, int u0, int rw, int nrw) {
    const int I = c.p->I;
    const uint32_t row_bytes = (uint32_t)c.p->H * sizeof(T);
    return [=](int s) -> uint32_t {
      const int br = rw + nrw * s;
      return (uint32_t)((br & 1) * I + u0 * EPW + (br >> 1)) * row_bytes;
    };
  }

  // ---------------------------------------------------------------- phase D
  // Units of EPW output rows; block b gets units [u0, u1); block row k goes
  // to role wave k % nrw.
  __device__ __forceinline__ static void d_range(const Ctx& c, int& u0, int& u1) {
    const int nu = c.p->H / EPW;
    u0 = c.b * nu / c.nb;
    u1 = (c.b + 1) * nu / c.nb;
  }
  __device__ __forceinline__ static Rows d_q(const Ctx& c, const LoopLayerW& lw, int nrows, int rw, int nrw) {
    const int my = rw < nrows ? (nrows - 1 - rw) / nrw + 1 : 0;
    return make_rows(lw.wdown, (int64_t)c.p->H * c.p->I * sizeof(T), c.p->I / VEC, my);
  }
  __device__ __forceinline__ static auto d_rows(const Ctx& c, int u0, int rw, int nrw) {
    const uint32_t row_bytes = (uint32_t)c.p->I * sizeof(T);
    return [=](int s) -> uint32_t { return (uint32_t)(u0 * EPW + rw + nrw * s) * row_bytes; };
  }

  // ---------------------------------------------------------------- LM head
  // Block b gets rows [r0, r1) of V; row r0 + k goes to weight wave k % NCW.
  __device__ __forceinline__ static void lm_range(const Ctx& c, int& r0, int& r1) {
    r0 = c.b * c.p->V / c.nb;
    r1 = (c.b + 1) * c.p->V / c.nb;
  }
  __device__ __forceinline__ static Rows lm_q(const Ctx& c, int nrows) {
    const int my = c.cw >= 0 && c.cw < nrows ? (nrows - 1 - c.cw) / NCW + 1 : 0;
    return make_rows(c.p->lm_head, (int64_t)c.p->V * c.p->H * sizeof(T), c.p->H / VEC, my);
  }
  __device__ __forceinline__ static auto lm_rows(const Ctx& c, int r0) {
    const int cw = c.cw;
    const uint32_t row_bytes = (uint32_t)c.p->H * sizeof(T);
    return [=](int s) -> uint32_t { return (uint32_t)(r0 + cw + NCW * s) * row_bytes; };
  }

  // ---------------------------------------------------------------- attention
  // LDS of the attention: a K and a V tile of TP cached positions (16-byte
  // pieces, piece c of row r at slot r * PPR + (c ^ (r % PPR)) so that
  // neither row-parallel nor column-parallel reads collide on banks), the
  // group's q rows (packed T), the current position's k and v (fp32) and the
  // scores of a tile.
  struct AttnLds {
    char* kt;   // [TP][PPR] 16-byte slots
    char* vt;   // [TP][PPR]
    T* q;       // [GMAXL][D]
    float* kn;  // [D]
    float* vn;  // [D]
    float* sc;  // [GMAXL][TP]
  };

  // Copy cached rows [p0, p0 + np) of the group's K and V into the tiles,
  // global -> LDS without registers. Wave-instruction j moves slots
  // [64 j, 64 j + 64); instructions are dealt to waves w0, w0 + 1, ... < w1.
  __device__ __forceinline__ static void tile_load(const Ctx& c, const T* kc, const T* vc, int p0, int np,
                                                   const AttnLds& s, int w0, int w1) {
    const int nins = (np * PPR + 63) / 64;
    for (int j = c.wave - w0; j < 2 * nins; j += w1 - w0) {
      const bool is_v = j >= nins;
      const int jj = is_v ? j - nins : j;
      const int slot = jj * 64 + c.lane;
      const int r = slot / PPR, cs = slot % PPR;
      const int piece = cs ^ (r % PPR);
      const T* src = (is_v ? vc : kc) + (int64_t)(p0 + (r < np ? r : 0)) * D + piece * VEC;
      char* dst = (is_v ? s.vt : s.kt) + jj * 1024;
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)dst, 16, 0, 0);
    }
  }

  // GQA attention of the block's KV group g for its G query heads over
  // ctx = cache_len + 1 positions: cached rows from K / V tiles in LDS (the
  // first tile was loaded during phase A), the current row from s.kn / s.vn.
  // Per tile, threads score one position against every head; then wave h
  // runs head h's online softmax over the tile and its P V (lane = dims).
  // The output, rounded to T, goes to xin (the o_proj input).
  __device__ __forceinline__ static void attention(const Ctx& c, int layer, int g, const AttnLds& s, T* xin,
                                                   bool tile_loader, int trs) {
    const LoopParams& p = *c.p;
    const int G = p.G;
    const int cached = (int)p.cache_len;
    const int64_t lay = (int64_t)layer * p.Hkv * p.S * D + (int64_t)g * p.S * D;
    const T* kc = (const T*)p.k_cache + lay;
    const T* vc = (const T*)p.v_cache + lay;
    const int h = c.wave;  // the head this wave owns in softmax and P V
    const int pg = c.lane / LPR, dc = c.lane % LPR;
    float m = -__builtin_inff(), l = 0.f, acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
    const uint4* q4 = (const uint4*)s.q;
    for (int p0 = 0; p0 < cached; p0 += TP) {
      const int np = cached - p0 < TP ? cached - p0 : TP;
      if (p0 > 0) {
        bar();  // every wave is done with the previous tile
        if (tile_loader) {  // the o_proj wave(s)
          tile_load(c, kc, vc, p0, np, s, p.role[1], p.role[2]);
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        bar();
      }
      // ---- scores of the tile: thread = position, every head
      for (int r = c.tid; r < np; r += LT) {
        float a[GMAXL];
#pragma unroll
        for (int hh = 0; hh < GMAXL; ++hh) a[hh] = 0.f;
        const uint4* krow = (const uint4*)(s.kt + r * PPR * 16);
#pragma unroll
        for (int pc = 0; pc < PPR; ++pc) {
          const uint4 kv = krow[pc ^ (r % PPR)];
#pragma unroll
          for (int hh = 0; hh < GMAXL; ++hh)
            if (hh < G) a[hh] = dot16<T>(kv, q4[hh * PPR + pc], a[hh]);
        }
#pragma unroll
        for (int hh = 0; hh < GMAXL; ++hh)
          if (hh < G) s.sc[hh * TP + r] = a[hh] * p.scale;
      }
      bar();
      c.mark(trs + LOOP_TR_ATT_SC);
      // ---- head h: online softmax over the tile, then P V
      if (h < G) {
        float* sh = s.sc + h * TP;
        float mx = -__builtin_inff();
        for (int r = c.lane; r < np; r += 64) mx = fmaxf(mx, sh[r]);
        const float mn = fmaxf(m, wave_max(mx));
        const float alpha = expf(m - mn);
        float ls = 0.f;
        for (int r = c.lane; r < np; r += 64) {
          const float pr = expf(sh[r] - mn);
          sh[r] = pr;
          ls += pr;
        }
        l = fmaf(l, alpha, wave_sum(ls));
        m = mn;
        wave_lds_fence();
        // P V: lane (row group pg, 8-element slice dc) walks rows pg, pg + RPI, ...
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll 4
        for (int r = pg; r < np; r += RPI) {
          const float pr = sh[r];
          float vf[8];
          const char* vrow = s.vt + r * PPR * 16;
          if constexpr (sizeof(T) == 2) {
            unpack16(*(const uint4*)(vrow + ((dc ^ (r % PPR)) * 16)), vf, (bf16*)nullptr);
          } else {
            unpack16(*(const uint4*)(vrow + (((2 * dc) ^ (r % PPR)) * 16)), vf, (float*)nullptr);
            unpack16(*(const uint4*)(vrow + (((2 * dc + 1) ^ (r % PPR)) * 16)), vf + 4, (float*)nullptr);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] = fmaf(pr, vf[e], acc[e]);
        }
      }
    }
    c.mark(trs + LOOP_TR_ATT_PV);
    // ---- the current position (its k and v came through the hand-off)
    if (h < G) {
      // sum the row groups: lanes sharing dc
#pragma unroll
      for (int msk = LPR; msk < 64; msk <<= 1)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], msk, 64);
      float sp = 0.f;
      for (int d = c.lane; d < D; d += 64) sp = fmaf(load_f32<T>(s.q, h * D + d), s.kn[d], sp);
      const float sv = wave_sum(sp) * p.scale;
      const float mn = fmaxf(m, sv);
      const float alpha = expf(m - mn);
      const float pr = expf(sv - mn);
      l = fmaf(l, alpha, pr);
      if (pg == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = dc * 8 + e;
          store_f32<T>(xin, h * D + d, fmaf(pr, s.vn[d], acc[e] * alpha) / l);
        }
      }
    }
    bar();
  }

  // ---------------------------------------------------------------- kernel body
  __device__ __forceinline__ static void run(const LoopParams& p) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    Ctx c;
    c.p = &p;
    c.b = blockIdx.x;
    c.nb = gridDim.x;
    c.tid = threadIdx.x;
    c.lane = c.tid & 63;
    c.wave = __builtin_amdgcn_readfirstlane(c.tid >> 6);  // wave-uniform: keep it scalar
    c.cw = c.wave - 1;
    {
      uint32_t e = p.ctrl[LOOP_CTRL_EPOCH] + 1u;
      c.epoch = e == 0u ? 1u : e;
    }
    float* xs = (float*)(lds + p.lds_xs);                 // residual stream x, fp32 holding T values
    T* xin = (T*)(lds + p.lds_xin);                       // GEMV input vector
    uint64_t* stage = (uint64_t*)(lds + p.lds_stage);    // gathered hand-off words
    uint64_t* qstage = (uint64_t*)(lds + p.lds_qstage);  // the group's q / k / v words
    float* rowres = (float*)(lds + p.lds_rowres);
    T* nws = (T*)(lds + p.lds_norm);          // the current RMSNorm weight
    float* red = (float*)(lds + p.lds_misc);  // [LWAVES]
    float* amv = red + LWAVES;                // [LWAVES]
    int64_t* ami = (int64_t*)(lds + p.lds_misc + 64 * 4);
    AttnLds at;  // K / V tiles in their own region; the rest aliases stage (free in phase B)
    at.kt = lds + p.lds_tile;
    at.vt = at.kt + TP * PPR * 16;
    at.q = (T*)(lds + p.lds_stage);
    at.kn = (float*)(at.q + GMAXL * D);
    at.vn = at.kn + D;
    at.sc = at.vn + D;
    const int H = p.H, Hq = p.Hq, Hkv = p.Hkv, G = p.G;
    const uint4* xin4 = (const uint4*)xin;

    // this wave's role: 0 = hand-offs, 1 = QKV, 2 = o_proj (+ K / V tiles),
    // 3 = gate/up, 4 = down weights
    const int role = c.wave == 0 ? 0 : c.wave < p.role[1] ? 1 : c.wave < p.role[2] ? 2 : c.wave < p.role[3] ? 3 : 4;
    const bool w0 = role == 0;
    const int rw = role == 0 ? 0 : c.wave - p.role[role - 1];     // index within the role
    const int nr = role == 0 ? 1 : p.role[role] - p.role[role - 1];  // waves in the role

    const int npb = a_pairs_block(c);
    int bg, br0, br1;
    b_rows_range(c, bg, br0, br1);
    const bool b_work = br1 > br0;
    const int bn = b_work ? br1 - br0 : 0;
    int cu0, cu1, du0, du1, lr0, lr1;
    c_range(c, cu0, cu1);
    d_range(c, du0, du1);
    lm_range(c, lr0, lr1);
    const int c_rows_n = 2 * EPW * (cu1 - cu0);
    const int d_rows_n = EPW * (du1 - du0);

    // Issue this wave's weight stream of a layer (roles 1..4).
    uint4 buf[BUFW];
    auto issue_a = [&](const LoopLayerW& w) {
      rows_issue<JA, SA>(buf, a_q(c, w, npb, rw, nr), a_rows(c, rw, nr), 0, 0, c.lane);
    };
    auto issue_b = [&](const LoopLayerW& w) {
      rows_issue<JB, SB>(buf, b_q(c, w, bg, bn, rw, nr), b_rows(c, br0, rw, nr), 0, 0, c.lane);
    };
    auto issue_c = [&](const LoopLayerW& w) {
      rows_issue<JC, SC>(buf, c_q(c, w, c_rows_n, rw, nr), c_rows(c, cu0, rw, nr), 0, 0, c.lane);
    };
    auto issue_d = [&](const LoopLayerW& w) {
      rows_issue<JD, SD>(buf, d_q(c, w, d_rows_n, rw, nr), d_rows(c, du0, rw, nr), 0, 0, c.lane);
    };
    // the o_proj wave(s) copy a layer's first K / V tile into LDS one layer
    // ahead (rows below cache_len were written by earlier steps)
    auto tile_next = [&](int layer) {
      if (b_work) {
        const int64_t lay_kv = (int64_t)layer * Hkv * p.S * D + (int64_t)bg * p.S * D;
        const int np0 = (int)(p.cache_len < TP ? p.cache_len : TP);
        tile_load(c, (const T*)p.k_cache + lay_kv, (const T*)p.v_cache + lay_kv, 0, np0, at, p.role[1], p.role[2]);
      }
    };
    if (role == 1) issue_a(p.layers[0]);
    if (role == 2) {
      tile_next(0);
      issue_b(p.layers[0]);
    }
    if (role == 3) issue_c(p.layers[0]);
    if (role == 4) issue_d(p.layers[0]);

    // ---- embedding (embedding.py:44-46): every block gathers the row. Only
    // wave 0 issues plain global loads: in waves 1..7 they would complete
    // behind the streamed weights.
    if (w0) {
      const int64_t id = p.ids[0];
      const bool ok = id >= 0 && id < p.V;
      const T* row = (const T*)p.embed + (ok ? id : 0) * H;
      for (int i = c.lane; i < H; i += 64) xs[i] = ok ? load_f32<T>(row, i) : __builtin_nanf("");
    }
    c.mark(LOOP_TR_START);
    const int64_t pos = p.positions[0];
    const bool pos_ok = pos >= 0 && pos < p.max_pos;
    if (!pos_ok && c.b == 0 && c.tid == 0)
      __hip_atomic_fetch_or(&p.ctrl[LOOP_CTRL_ERROR], (uint32_t)LOOP_ERR_POSITION, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);

    for (int layer = 0; layer < p.L; ++layer) {
      const LoopLayerW& lw = p.layers[layer];
      const bool more = layer + 1 < p.L;
      const LoopLayerW& nw = p.layers[more ? layer + 1 : layer];
      const int tr = 1 + layer * LOOP_TR_PER_LAYER;
      uint64_t* ll = p.ll + (int64_t)layer * p.ll_layer_words;
      uint64_t* ll_qkv = ll + p.off_qkv;
      uint64_t* ll_p = ll + p.off_p;
      uint64_t* ll_act = ll + p.off_act;
      uint64_t* ll_down = ll + p.off_down;

      // ======== A: x += down (previous layer), RMSNorm, QKV + RoPE ========
      if (w0) {
        lds_fetch(c, lw.ln1, H * (int)sizeof(T), nws);
        if (layer > 0)
          ll_gather(c, p.ll + (int64_t)(layer - 1) * p.ll_layer_words + p.off_down, H / EPW, stage);
        else
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the norm weight
      }
      bar();
      if (layer > 0) {
        for (int i = c.tid; i < H; i += LT)
          xs[i] = round_to<T>(add_rn(xs[i], word_elem<T>(payload(stage[i / EPW]), i % EPW)));
        bar();
      }
      c.mark(tr + LOOP_TR_A_IN);
      // wave 0: this phase's epilogue inputs (bias, RoPE rows), ahead of use
      float eb[2] = {0.f, 0.f}, ecs[4] = {0.f, 0.f, 0.f, 0.f};
      if (w0 && c.lane < npb) {
        const int pr = c.b + c.nb * c.lane;
        const int hd = pr / HALF, i = pr % HALF;
        eb[0] = load_f32<T>((const T*)lw.bqkv, hd * D + i);
        eb[1] = load_f32<T>((const T*)lw.bqkv, hd * D + i + HALF);
        if (pos_ok && hd < Hq + Hkv) {
          ecs[0] = p.cos_tab[pos * D + i];
          ecs[1] = p.sin_tab[pos * D + i];
          ecs[2] = p.cos_tab[pos * D + i + HALF];
          ecs[3] = p.sin_tab[pos * D + i + HALF];
        }
      }
      block_rmsnorm<T>(c, xs, nws, xin, red);
      if (role == 1) {
        rows_consume<T, JA, SA>(buf, a_q(c, lw, npb, rw, nr), a_rows(c, rw, nr), xin4, c.lane, [&](int s, float v) {
          if (c.lane == 0) rowres[2 * (rw + nr * (s >> 1)) + (s & 1)] = v;
        });
      }
      bar();
      if (w0 && c.lane < npb) {  // npb <= 64
        const int t = c.lane;
        const int pr = c.b + c.nb * t;
        const int hd = pr / HALF, i = pr % HALF;
        // F.linear output with bias, rounded to the dtype (fused.py:58)
        const float va = round_to<T>(add_rn(rowres[2 * t], eb[0]));
        const float vb = round_to<T>(add_rn(rowres[2 * t + 1], eb[1]));
        float o[2] = {va, vb};
        if (hd < Hq + Hkv) {
          // rotate: x * cos + rotate_half(x) * sin, fp32, each op rounded,
          // then cast (rope.py:57-62)
          if (pos_ok) {
            o[0] = round_to<T>(add_rn(mul_rn(va, ecs[0]), -mul_rn(vb, ecs[1])));
            o[1] = round_to<T>(add_rn(mul_rn(vb, ecs[2]), mul_rn(va, ecs[3])));
          } else {
            o[0] = o[1] = __builtin_nanf("");
          }
        }
        uint64_t* wq = ll_qkv + qkv_word(c, hd, i);
        if constexpr (EPW == 2) {
          ll_store(wq, c.epoch, pack_word<T>(o));
        } else {
          ll_store(wq, c.epoch, pack_word<T>(&o[0]));
          ll_store(wq + 1, c.epoch, pack_word<T>(&o[1]));
        }
        if (hd >= Hq) {  // KV cache row at cache_len (kv_cache.py:53-54)
          const bool is_k = hd < Hq + Hkv;
          const int gg = is_k ? hd - Hq : hd - Hq - Hkv;
          T* cache = (T*)(is_k ? p.k_cache : p.v_cache) +
                     ((int64_t)layer * Hkv * p.S + (int64_t)gg * p.S + p.cache_len) * D;
          store_f32<T>(cache, i, o[0]);
          store_f32<T>(cache, i + HALF, o[1]);
        }
      }
      c.mark(tr + LOOP_TR_A_OUT);
      if (role == 1 && more) issue_a(nw);  // overlaps the hand-off to phase B
      c.mark(tr + LOOP_TR_A_ISSUED);

      // ======== B: attention of group bg + its o_proj share for rows [br0, br1) ========
      if (b_work) {
        if (w0) {
          const int gw = (G + 2) * HALF * WPP;  // the group's q heads, k head, v head
          ll_gather(c, ll_qkv + (int64_t)bg * gw, gw, qstage);
        } else if (role == 2) {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the K / V tile
        }
        bar();
        for (int t = c.tid; t < (G + 2) * HALF; t += LT) {
          const int hh = t / HALF, i = t % HALF;
          float va, vb;
          if constexpr (EPW == 2) {
            const uint32_t w = payload(qstage[t]);
            va = word_elem<T>(w, 0);
            vb = word_elem<T>(w, 1);
          } else {
            va = __uint_as_float(payload(qstage[2 * t]));
            vb = __uint_as_float(payload(qstage[2 * t + 1]));
          }
          if (hh < G) {
            store_f32<T>(at.q, hh * D + i, va);
            store_f32<T>(at.q, hh * D + i + HALF, vb);
          } else {
            float* dst = hh == G ? at.kn : at.vn;
            dst[i] = va;
            dst[i + HALF] = vb;
          }
        }
        bar();
        c.mark(tr + LOOP_TR_B_IN);
        attention(c, layer, bg, at, xin, role == 2, tr);
        c.mark(tr + LOOP_TR_B_ATTN);
        if (role == 2)
          rows_consume<T, JB, SB>(buf, b_q(c, lw, bg, bn, rw, nr), b_rows(c, br0, rw, nr), xin4, c.lane,
                                  [&](int s, float v) {
                                    if (c.lane == 0) rowres[rw + nr * s] = v;
                                  });
        bar();
        if (w0)
          for (int t = c.lane; t < bn; t += 64)
            ll_store(ll_p + (int64_t)bg * H + br0 + t, c.epoch, __float_as_uint(rowres[t]));
        c.mark(tr + LOOP_TR_B_OUT);
      }
      if (role == 2 && more) {  // overlaps the hand-off to phase C
        tile_next(layer + 1);
        issue_b(nw);
      }
      c.mark(tr + LOOP_TR_B_ISSUED);

      // ======== C: x += dtype(o_proj), RMSNorm, gate/up, SwiGLU ========
      if (w0) {
        lds_fetch(c, lw.ln2, H * (int)sizeof(T), nws);
        ll_gather(c, ll_p, Hkv * H, stage);
      }
      bar();
      c.mark(tr + LOOP_TR_C_IN);
      for (int i = c.tid; i < H; i += LT) {
        float o = 0.f;
        for (int g = 0; g < Hkv; ++g) o += __uint_as_float(payload(stage[g * H + i]));
        xs[i] = round_to<T>(add_rn(xs[i], round_to<T>(o)));
      }
      bar();
      block_rmsnorm<T>(c, xs, nws, xin, red);
      if (role == 3) {
        rows_consume<T, JC, SC>(buf, c_q(c, lw, c_rows_n, rw, nr), c_rows(c, cu0, rw, nr), xin4, c.lane,
                                [&](int s, float v) {
                                  if (c.lane == 0) rowres[rw + nr * s] = v;
                                });
      }
      bar();
      if (w0) {
        for (int t = c.lane; t < cu1 - cu0; t += 64) {
          float a[EPW];
#pragma unroll
          for (int e = 0; e < EPW; ++e) {
            const int br = 2 * (t * EPW + e);
            a[e] = swiglu<T>(round_to<T>(rowres[br]), round_to<T>(rowres[br + 1]));  // mlp.py:38
          }
          ll_store(ll_act + cu0 + t, c.epoch, pack_word<T>(a));
        }
      }
      c.mark(tr + LOOP_TR_C_OUT);
      if (role == 3 && more) issue_c(nw);  // overlaps the hand-off to phase D
      c.mark(tr + LOOP_TR_C_ISSUED);

      // ======== D: down projection ========
      if (d_rows_n > 0) {
        if (w0) ll_gather(c, ll_act, p.I / EPW, stage);
        bar();
        for (int i = c.tid; i < p.I / EPW; i += LT) ((uint32_t*)xin)[i] = payload(stage[i]);
        bar();
        c.mark(tr + LOOP_TR_D_IN);
        if (role == 4)
          rows_consume<T, JD, SD>(buf, d_q(c, lw, d_rows_n, rw, nr), d_rows(c, du0, rw, nr), xin4, c.lane,
                                  [&](int s, float v) {
                                    if (c.lane == 0) rowres[rw + nr * s] = v;
                                  });
        bar();
        if (w0) {
          for (int t = c.lane; t < du1 - du0; t += 64) {
            float o[EPW];
#pragma unroll
            for (int e = 0; e < EPW; ++e) o[e] = round_to<T>(rowres[t * EPW + e]);
            ll_store(ll_down + du0 + t, c.epoch, pack_word<T>(o));
          }
        }
        c.mark(tr + LOOP_TR_D_OUT);
      }
      if (role == 4 && more) issue_d(nw);
      c.mark(tr + LOOP_TR_D_ISSUED);
    }

    // ======== final norm, LM head, greedy pick ========
    {
      const int tr = 1 + p.L * LOOP_TR_PER_LAYER;
      // the LM head streams through every weight wave
      if (!w0) rows_issue<JL, SL>(buf, lm_q(c, lr1 - lr0), lm_rows(c, lr0), 0, 0, c.lane);
      if (w0) {
        lds_fetch(c, p.final_norm, H * (int)sizeof(T), nws);
        ll_gather(c, p.ll + (int64_t)(p.L - 1) * p.ll_layer_words + p.off_down, H / EPW, stage);
      }
      bar();
      c.mark(tr);
      for (int i = c.tid; i < H; i += LT)
        xs[i] = round_to<T>(add_rn(xs[i], word_elem<T>(payload(stage[i / EPW]), i % EPW)));
      bar();
      block_rmsnorm<T>(c, xs, nws, xin, red);
      if (!w0) {
        const int cw = c.cw;
        rows_consume<T, JL, SL>(buf, lm_q(c, lr1 - lr0), lm_rows(c, lr0), xin4, c.lane, [&](int s, float v) {
          if (c.lane == 0) rowres[cw + NCW * s] = v;
        });
      }
      bar();
      float bv = -__builtin_inff();
      int64_t bi = INT64_MAX;
      T* logits = (T*)p.logits;
      for (int t = c.tid; t < lr1 - lr0; t += LT) {
        const float v = round_to<T>(rowres[t]);
        if (logits) store_f32<T>(logits, lr0 + t, v);
        if (argmax_better(v, lr0 + t, bv, bi)) {
          bv = v;
          bi = lr0 + t;
        }
      }
      block_argmax(c, bv, bi, amv, ami);
      c.mark(tr + 1);
      uint64_t* part = p.ll + p.off_lm;
      if (c.tid == 0) {
        ll_store(part + 2 * c.b, c.epoch, __float_as_uint(amv[0]));
        ll_store(part + 2 * c.b + 1, c.epoch, (uint32_t)ami[0]);
      }
      if (c.b == 0) {
        if (w0) ll_gather(c, part, 2 * c.nb, stage);
        bar();
        float v = -__builtin_inff();
        int64_t i = INT64_MAX;
        if (c.tid < c.nb) {
          v = __uint_as_float(payload(stage[2 * c.tid]));
          i = (int64_t)payload(stage[2 * c.tid + 1]);
        }
        block_argmax(c, v, i, amv, ami);
        if (c.tid == 0) {
          if (p.next_tok) p.next_tok[0] = ami[0];
          p.ctrl[LOOP_CTRL_EPOCH] = c.epoch;
        }
        c.mark(tr + 2);
      }
    }
  }
};

template <typename T, int D>
__global__ __launch_bounds__(LT) void decode_loop_kernel(LoopParams p) {
  Loop<T, D>::run(p);
}

template <typename T>
const void* pick_kernel(int D) {
#ifdef LOOP_PROBE_ONLY
  if (D == 64) return (const void*)decode_loop_kernel<T, 64>;
  return nullptr;
#else
  switch (D) {
    case 16:
      return (const void*)decode_loop_kernel<T, 16>;
    case 32:
      return (const void*)decode_loop_kernel<T, 32>;
    case 64:
      return (const void*)decode_loop_kernel<T, 64>;
    case 128:
      return (const void*)decode_loop_kernel<T, 128>;
  }
  return nullptr;
#endif
}

inline int align_up(int v, int a) { return (v + a - 1) / a * a; }

}  // namespace

const void* loop_kernel(int dtype, int D) {
#ifdef LOOP_PROBE_ONLY
  return dtype == MINITP_F32 ? nullptr : pick_kernel<bf16>(D);
#else
  return dtype == MINITP_F32 ? pick_kernel<float>(D) : pick_kernel<bf16>(D);
#endif
}

// LL words of one layer and their offsets; the same for every device.
LoopLayout loop_layout(const minitp_qwen2_config& c) {
  LoopLayout L{};
  const int epw = c.dtype == MINITP_F32 ? 1 : 2;
  const int wpp = 2 / epw;
  L.off_qkv = 0;
  L.off_p = align_up((c.heads + 2 * c.kv_heads) * (c.head_dim / 2) * wpp, 64);
  L.off_act = L.off_p + align_up(c.kv_heads * c.hidden, 64);
  L.off_down = L.off_act + align_up(c.intermediate / epw, 64);
  L.layer_words = L.off_down + align_up(c.hidden / epw, 64);
  L.off_lm = (int64_t)L.layer_words * c.num_layers;
  L.total_words = L.off_lm + 2 * LOOP_MAX_BLOCKS;
  L.bytes = LOOP_CTRL_BYTES + L.total_words * 8;
  return L;
}

// Split the weight-streaming waves between the four phases in proportion to
// the bytes each phase streams per block (at least one wave each): out[0..4]
// are the wave boundaries (role[0] = 1, role[4] = LWAVES).
void loop_roles(const minitp_qwen2_config& c, int nb, int* out) {
  const double es = c.dtype == MINITP_F32 ? 4.0 : 2.0;
  const double H = c.hidden, I = c.intermediate, D = c.head_dim;
  const double rs = nb / c.kv_heads;
  const double bytes[4] = {(c.heads + 2.0 * c.kv_heads) * D * H * es / nb,       // QKV
                           (H / rs) * (c.heads / c.kv_heads) * D * es,           // o_proj share
                           2.0 * I * H * es / nb,                                // gate/up
                           H * I * es / nb};                                     // down
  int n[4] = {1, 1, 1, 1};
  for (int left = NCW - 4; left > 0; --left) {
    int k = 0;
    for (int j = 1; j < 4; ++j)
      if (bytes[j] / n[j] > bytes[k] / n[k]) k = j;
    ++n[k];
  }
  out[0] = 1;
  for (int j = 0; j < 4; ++j) out[j + 1] = out[j] + n[j];
}

// Why the persistent decode cannot serve this model (nullptr: it can), and
// the LDS layout when it can.
const char* loop_unsupported(const minitp_qwen2_config& c, int nb, LoopLds* out) {
  const int D = c.head_dim;
  if (D != 16 && D != 32 && D != 64 && D != 128) return "head_dim not in {16, 32, 64, 128}";
  if (c.heads % c.kv_heads != 0 || c.heads / c.kv_heads > GMAXL) return "more than 8 query heads per KV head";
  const int es = c.dtype == MINITP_F32 ? 4 : 2;
  const int vec = 16 / es;
  if (c.hidden % vec || c.intermediate % vec || (c.heads / c.kv_heads * D) % vec) return "row length not whole 16 B";
  if (c.intermediate % 2 || c.hidden % 2) return "odd hidden / intermediate";
  if (nb < c.kv_heads || nb > LOOP_MAX_BLOCKS) return "grid size";
  {
    const int64_t e = c.dtype == MINITP_F32 ? 4 : 2;
    const int64_t big = std::max(std::max((int64_t)c.vocab * c.hidden, (int64_t)2 * c.intermediate * c.hidden),
                                 (int64_t)(c.heads + 2 * c.kv_heads) * c.head_dim * c.hidden);
    if (big * e >= ((int64_t)1 << 31)) return "a weight matrix of 2 GiB or more (buffer-load range)";
  }
  const int G = c.heads / c.kv_heads;
  int tp = ATT_KV_BYTES / 2 / (D * es);
  if (tp > 256) tp = 256;
  LoopLds L{};
  int off = 0;
  auto take = [&](int bytes) {
    int r = off;
    off = align_up(off + bytes, 16);
    return r;
  };
  L.xs = take(c.hidden * 4);
  const int xin_elems = std::max(std::max(c.hidden, c.intermediate), G * D);
  L.xin = take(align_up(xin_elems * es, 16) + 16);
  // attention: K and V tiles (own region), q rows, current k and v, tile scores (in stage)
  L.tile = take(2 * tp * D * es);
  const int attn_bytes = GMAXL * D * es + 2 * D * 4 + GMAXL * tp * 4;
  // gathered hand-off words (8 bytes each, whole 128-word copies)
  const int epw_ = es == 4 ? 1 : 2;
  const int gmax = std::max(std::max(c.kv_heads * c.hidden, c.hidden / epw_), std::max(c.intermediate / epw_, 2 * nb));
  if (gmax > 64 * 128) return "a hand-off exceeds 8192 words";
  const int stage_words = align_up(gmax, 128);
  L.stage = take(std::max(attn_bytes, stage_words * 8));
  L.qstage = take(align_up((G + 2) * (D / 2) * (2 / epw_), 128) * 8);
  // row results: phase A 2 * pairs, B rows, C rows, D NCW * rows, LM rows
  const int npa = (c.heads + 2 * c.kv_heads) * (D / 2);
  const int rs = nb / c.kv_heads;
  const int rows_a = 2 * ((npa + nb - 1) / nb);
  const int rows_b = (c.hidden + rs - 1) / rs;
  const int epw = es == 4 ? 1 : 2;
  const int rows_c = 2 * epw * ((c.intermediate / epw + nb - 1) / nb);
  const int rows_d = NCW * epw * ((c.hidden / epw + nb - 1) / nb);
  const int rows_lm = (c.vocab + nb - 1) / nb;
  L.rowres = take(std::max(std::max(std::max(rows_a, rows_b), std::max(rows_c, rows_d)), rows_lm) * 4 + 16);
  L.norm = take(align_up(c.hidden * es, 1024));
  L.misc = take(64 * 4 + LWAVES * 8);
  if ((npa + nb - 1) / nb > 64) return "more than 64 QKV pairs per block";
  L.bytes = off;
  if (L.bytes > 160 * 1024) return "LDS layout exceeds 160 KiB";
  if (out) *out = L;
  return nullptr;
}

}  // namespace minitp
