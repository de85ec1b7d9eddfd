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
// Inside a block (8 waves): wave 0 is the only wave that waits on hand-off
// words (it copies them global -> LDS with global_load_lds_dwordx4 and
// re-reads only the copies still holding an older epoch); it also copies
// the norm weights and the K / V rows of the block's KV group into LDS.
// Waves 1..7 hold every phase's rows of the NEXT layer in registers
// (buffer loads, issued after the current layer's results of that phase are
// stored; the gate/up and down batches in three parts over three phases),
// so weight latency stays off the critical path. All eight waves share the
// glue (residual add + RMSNorm, one 4-element group per thread) and the
// attention (scores and P V on MFMA 16x16x16 for bf16), meeting at
// s_barrier; a weight wave's results go straight from its registers to its
// hand-off words.
//
// Measured on MI355X at the 0.5B shape this path is slower than the graph of
// per-op kernels: the hand-offs cost 2-7 us each, mostly waiting behind the
// CU's own weight loads in the vector-memory queue, so it stays opt-in
// (MINITP_DECODE_PERSISTENT).
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
constexpr int JA = 2, SA = 2, JB = 1, SB = 2, JC = 2, SC = 8, JD = 10, SD = 1, JL = 2, SL = 14;
constexpr int LOOP_ROWS_PER_WAVE = 64;  // LDS row results per weight wave (phases A, C)
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
// Waits for every outstanding vector-memory operation of this wave, as an
// s_waitcnt the compiler sees: after it, the compiler knows that no LDS DMA
// (global_load_lds) is in flight, so it adds no waits of its own before
// later LDS reads in any wave (its analysis does not tell waves apart).
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)
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
    wait_vm0();
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
// the 16-byte chunks l, l + 64, ... (cpl of them) of every row (nch chunks),
// so one wave-instruction reads 1 KiB of a row contiguously and the LDS
// input vector is read the same way, free of bank conflicts. The buffer
// resource covers the matrix from `base` (bytes bytes;
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

// A register batch of a stream: J chunk columns x S slots, load (j, s) at
// index j * S + s.

// Issue the batch of slots [sb, sb + S) x columns [jb, jb + J). Every load
// is issued; loads outside the stream get an out-of-range lane offset and
// return zeros without touching memory, so the code has no branches.
// The buffer resource, built from wave-uniform values made explicitly
// uniform (otherwise the compiler may keep it in vector registers and wrap
// every load in a loop over distinct lane values).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const Rows& q) { return span_rsrc(q.base, (uint32_t)q.bytes); }

// Issue loads [T0, T1) of the batch of slots [sb, sb + S) x columns
// [jb, jb + J), load t being (slot t / J, column t % J): a batch can go out
// in parts, spread over time. Every load is issued; loads outside the
// stream get an out-of-range lane offset and return zeros without touching
// memory, so the code has no branches.
template <int J, int S, int T0, int T1, int N, class RowFn>
__device__ __forceinline__ void rows_issue_part(uint4 (&buf)[N], const Rows& q, RowFn row_off, int sb, int jb,
                                                int lane) {
  static_assert(J * S <= N, "batch larger than the register buffer");
  static_assert(0 <= T0 && T0 <= T1 && T1 <= J * S, "part outside the batch");
  if constexpr (T1 > T0) {
    const __amdgpu_buffer_rsrc_t rsrc = rows_rsrc(q);
    uint32_t vo[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int cc = (jb + j) * 64 + lane;
      vo[j] = cc < q.nch ? (uint32_t)cc * 16u : OFF_RANGE;
    }
#pragma unroll
    for (int s = T0 / J; s <= (T1 - 1) / J; ++s) {
      const bool live = sb + s < q.ns;
      const uint32_t so = __builtin_amdgcn_readfirstlane(live ? row_off(sb + s) : 0u);
#pragma unroll
      for (int j = 0; j < J; ++j) {
        if (s * J + j < T0 || s * J + j >= T1) continue;
        const u32x4v v = __builtin_bit_cast(
            u32x4v, __builtin_amdgcn_raw_buffer_load_b128(rsrc, live ? vo[j] : OFF_RANGE, so, 2 /* nt */));
        buf[j * S + s] = make_uint4(v.x, v.y, v.z, v.w);
      }
    }
  }
}
template <int J, int S, int N, class RowFn>
__device__ __forceinline__ void rows_issue(uint4 (&buf)[N], const Rows& q, RowFn row_off, int sb, int jb, int lane) {
  rows_issue_part<J, S, 0, J * S>(buf, q, row_off, sb, jb, lane);
}

// Dot every row of the stream with the LDS input x, batch by batch; the
// first batch (sb = 0, jb = 0) was issued by the caller. Hands each row's
// wave-reduced sum to done(slot, value) (executed by every lane).
template <typename T, int J, int S, int N, class RowFn, class DoneFn>
__device__ __forceinline__ void rows_consume(uint4 (&buf)[N], const Rows& q, RowFn row_off, const uint4* x,
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
        const int cc = (jb + j) * 64 + lane;
        xj[j] = cc < q.nch ? x[cc] : make_uint4(0, 0, 0, 0);
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
  static constexpr int RPW = LOOP_ROWS_PER_WAVE;     // per-wave row results in LDS (phases A, C)

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

  // The weight waves w = 1 .. NCW take every phase's rows, rw = w - 1 of
  // nrw = NCW. A stream built with live == false has no rows: its loads
  // return zeros without touching memory (the last layer's "next layer").

  // ---------------------------------------------------------------- phase A
  // Pair p = (head hd, dim i < D/2): rows hd * D + i and hd * D + i + D/2 of
  // the fused QKV weight (q heads, then k, then v; fused.py:60). Pair p goes
  // to block p % nb; local pair lp = p / nb to weight wave lp % nrw, whose
  // slots 2t, 2t + 1 are the two rows of its t-th pair.
  __device__ __forceinline__ static int a_pairs_block(const Ctx& c) {
    const int npa = (c.p->Hq + 2 * c.p->Hkv) * HALF;
    return c.b < npa ? (npa - 1 - c.b) / c.nb + 1 : 0;
  }
  __device__ __forceinline__ static int a_my(int npb, int rw, int nrw) {
    return rw < npb ? (npb - 1 - rw) / nrw + 1 : 0;
  }
  __device__ __forceinline__ static Rows a_q(const Ctx& c, const LoopLayerW& lw, int my, bool live) {
    return make_rows(lw.wqkv, (int64_t)(c.p->Hq + 2 * c.p->Hkv) * D * c.p->H * sizeof(T), c.p->H / VEC,
                     live ? 2 * my : 0);
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
  // (head, dim) of this wave's t-th pair
  __device__ __forceinline__ static void a_pair(const Ctx& c, int rw, int nrw, int t, int& hd, int& i) {
    const int p = c.b + c.nb * (rw + nrw * t);
    hd = p / HALF;
    i = p % HALF;
  }

  // ---------------------------------------------------------------- phase B
  // Block b < Hkv * RS serves KV group g = b % Hkv and output rows
  // [r0, r1) = slice b / Hkv of RS equal slices of H; row r0 + k goes to
  // weight wave k % nrw. The buffer starts at the group's first column of
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
  __device__ __forceinline__ static Rows b_q(const Ctx& c, const LoopLayerW& lw, int g, int nrows, int rw, int nrw,
                                             bool live) {
    const int my = rw < nrows ? (nrows - 1 - rw) / nrw + 1 : 0;
    const int64_t off = (int64_t)g * c.p->G * D;
    return make_rows((const T*)lw.wo + off, ((int64_t)c.p->H * c.p->Hq * D - off) * sizeof(T), c.p->G * D / VEC,
                     live ? my : 0);
  }
  __device__ __forceinline__ static auto b_rows(const Ctx& c, int r0, int rw, int nrw) {
    const uint32_t row_bytes = (uint32_t)c.p->Hq * D * sizeof(T);
    return [=](int s) -> uint32_t { return (uint32_t)(r0 + rw + nrw * s) * row_bytes; };
  }

  // ---------------------------------------------------------------- phase C
  // Units of EPW intermediate indices; block b gets units [u0, u1), unit
  // u0 + k to weight wave k % nrw. A wave's t-th unit fills slots
  // 2 EPW t .. 2 EPW t + 2 EPW - 1: slot 2 e + 0 / 1 is the gate / up row of
  // index (u0 + rw + nrw t) * EPW + e.
  __device__ __forceinline__ static void c_range(const Ctx& c, int& u0, int& u1) {
    const int nu = c.p->I / EPW;
    u0 = c.b * nu / c.nb;
    u1 = (c.b + 1) * nu / c.nb;
  }
  __device__ __forceinline__ static Rows c_q(const Ctx& c, const LoopLayerW& lw, int my_units, bool live) {
    return make_rows(lw.wgu, (int64_t)2 * c.p->I * c.p->H * sizeof(T), c.p->H / VEC, live ? 2 * EPW * my_units : 0);
  }
  __device__ __forceinline__ static auto c_rows(const Ctx& c, int u0, int rw, int nrw) {
    const int I = c.p->I;
    const uint32_t row_bytes = (uint32_t)c.p->H * sizeof(T);
    return [=](int s) -> uint32_t {
      const int t = s / (2 * EPW), k = s % (2 * EPW);
      return (uint32_t)((k & 1) * I + (u0 + rw + nrw * t) * EPW + (k >> 1)) * row_bytes;
    };
  }

  // ---------------------------------------------------------------- phase D
  // Units of EPW output rows; block b gets units [u0, u1); block row k goes
  // to weight wave k % nrw.
  __device__ __forceinline__ static void d_range(const Ctx& c, int& u0, int& u1) {
    const int nu = c.p->H / EPW;
    u0 = c.b * nu / c.nb;
    u1 = (c.b + 1) * nu / c.nb;
  }
  __device__ __forceinline__ static Rows d_q(const Ctx& c, const LoopLayerW& lw, int nrows, int rw, int nrw,
                                             bool live) {
    const int my = rw < nrows ? (nrows - 1 - rw) / nrw + 1 : 0;
    return make_rows(lw.wdown, (int64_t)c.p->H * c.p->I * sizeof(T), c.p->I / VEC, live ? my : 0);
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
    float* st;  // [4][GMAXL] softmax factors
  };

  // Wave 0: copy cached rows [p0, p0 + np) of the group's K and V into the
  // tiles, global -> LDS without registers; wave-instruction j moves slots
  // [64 j, 64 j + 64). The caller waits (wait_vm0) before the tiles are read.
  __device__ __forceinline__ static void tile_load(const Ctx& c, const T* kc, const T* vc, int p0, int np,
                                                   const AttnLds& s) {
    const int nins = (np * PPR + 63) / 64;
    for (int j = 0; j < 2 * nins; ++j) {
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

  // bf16 attention on matrix cores. Per tile: scores S = Q K^T by MFMA
  // 16x16x16 (rows = the group's q heads padded to 16, columns = 16
  // positions; wave w takes position blocks w, w + 8, ...), kept in LDS
  // pre-multiplied by scale * log2(e); wave h runs head h's online softmax in
  // base 2 over the tile, leaving P = 2^(S - m) in place and the factor that
  // rescales earlier tiles in s.st[h]; then O += P V by MFMA (rows = heads,
  // columns = 16 dims, inner = 16 positions; P rounded to bf16 as the MFMA
  // operand, accumulation in fp32), wave w owning dim block w % (D / 16) and
  // every (8 / (D / 16))-th position step. Finally the current position
  // (k, v from the hand-off) joins the softmax, the position-step partials
  // are summed through LDS and the output, rounded to bf16, goes to xin.
  __device__ __forceinline__ static void attention_mfma(const Ctx& c, int layer, int g, const AttnLds& s, T* xin,
                                                        int trs) {
    typedef short short4_t __attribute__((ext_vector_type(4)));
    typedef float float4_t __attribute__((ext_vector_type(4)));
    constexpr int KS = D / 16;                // 16-dim steps of a score
    constexpr int NBK = D / 16;               // 16-dim output blocks
    constexpr int KH = LWAVES / NBK;          // waves sharing an output block
    constexpr float LOG2E = 1.4426950408889634f;
    const LoopParams& p = *c.p;
    const int G = p.G;
    const int cached = (int)p.cache_len;
    const int64_t lay = (int64_t)layer * p.Hkv * p.S * D + (int64_t)g * p.S * D;
    const T* kc = (const T*)p.k_cache + lay;
    const T* vc = (const T*)p.v_cache + lay;
    const int lr = c.lane % 16, lq = c.lane / 16;
    const int nbk = c.wave % NBK, kh = c.wave / NBK;
    const float sl2 = p.scale * LOG2E;
    float* alpha_s = s.st;              // [GMAXL] rescale factor of the tile
    float* fin_a = s.st + GMAXL;        // [GMAXL] final factors
    float* fin_p = s.st + 2 * GMAXL;
    float* fin_l = s.st + 3 * GMAXL;
    // head h's running max and sum (wave h)
    float m = -__builtin_inff(), l = 0.f;
    float4_t o = {0.f, 0.f, 0.f, 0.f};  // O[4 lq + i][16 nbk + lr], partial over this wave's position steps
    short4_t qa[KS];
#pragma unroll
    for (int kb = 0; kb < KS; ++kb) {
      const uint2 v = lr < G ? *(const uint2*)(s.q + lr * D + kb * 16 + 4 * lq) : make_uint2(0, 0);
      qa[kb] = __builtin_bit_cast(short4_t, v);
    }
    for (int p0 = 0; p0 < cached; p0 += TP) {
      const int np = cached - p0 < TP ? cached - p0 : TP;
      if (p0 > 0) {
        bar();  // every wave is done with the previous tile
        if (c.wave == 0) {
          tile_load(c, kc, vc, p0, np, s);
          wait_vm0();
        }
        bar();
      }
      // ---- scores
      for (int blk = c.wave; blk * 16 < np; blk += LWAVES) {
        const int r = blk * 16 + lr;
        const char* krow = s.kt + r * PPR * 16;
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KS; ++kb) {
          const int piece = 2 * kb + (lq >> 1);
          const uint2 v = r < np ? *(const uint2*)(krow + ((piece ^ (r % PPR)) * 16) + (lq & 1) * 8) : make_uint2(0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(qa[kb], __builtin_bit_cast(short4_t, v), acc, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int hh = 4 * lq + i;
          if (hh < G && r < np) s.sc[hh * TP + r] = acc[i] * sl2;
        }
      }
      bar();
      c.mark(trs + LOOP_TR_ATT_SC);
      // ---- wave h: head h's softmax over the tile (base 2)
      if (c.wave < G) {
        float* sh = s.sc + c.wave * TP;
        float mx = -__builtin_inff();
        for (int r = c.lane; r < np; r += 64) mx = fmaxf(mx, sh[r]);
        const float mn = fmaxf(m, wave_max(mx));
        const float alpha = __builtin_amdgcn_exp2f(m - mn);
        float ls = 0.f;
        for (int r = c.lane; r < np; r += 64) {
          const float pr = __builtin_amdgcn_exp2f(sh[r] - mn);
          sh[r] = pr;
          ls += pr;
        }
        l = fmaf(l, alpha, wave_sum(ls));
        m = mn;
        if (c.lane == 0) alpha_s[c.wave] = alpha;
      }
      bar();
      // ---- O = O * alpha + P V over this wave's position steps
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int hh = 4 * lq + i;
        o[i] *= hh < G ? alpha_s[hh] : 1.f;
      }
      const int dcol = nbk * 16 + lr;  // this lane's output dim
      const int dpc = dcol / 8, dofs = (dcol % 8) * 2;
      for (int ks = kh; ks * 16 < np; ks += KH) {
        const int k0 = ks * 16 + 4 * lq;  // this lane's 4 positions
        float4 pv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (lr < G) pv = *(const float4*)(s.sc + lr * TP + k0);
        const float pp[4] = {pv.x, pv.y, pv.z, pv.w};
        uint32_t pa[2], vb[2];
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          const float a0 = k0 + e < np ? pp[e] : 0.f, a1 = k0 + e + 1 < np ? pp[e + 1] : 0.f;
          pa[e / 2] = (uint32_t)f32_to_bf16(a0) | ((uint32_t)f32_to_bf16(a1) << 16);
          uint32_t v0 = 0, v1 = 0;
          const int r0 = k0 + e, r1 = k0 + e + 1;
          if (r0 < np) v0 = *(const uint16_t*)(s.vt + r0 * PPR * 16 + ((dpc ^ (r0 % PPR)) * 16) + dofs);
          if (r1 < np) v1 = *(const uint16_t*)(s.vt + r1 * PPR * 16 + ((dpc ^ (r1 % PPR)) * 16) + dofs);
          vb[e / 2] = v0 | (v1 << 16);
        }
        o = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_t, make_uint2(pa[0], pa[1])),
                                                      __builtin_bit_cast(short4_t, make_uint2(vb[0], vb[1])), o, 0, 0,
                                                      0);
      }
    }
    c.mark(trs + LOOP_TR_ATT_PV);
    // ---- the current position (its k and v came through the hand-off)
    if (c.wave < G) {
      float sp = 0.f;
      for (int d = c.lane; d < D; d += 64) sp = fmaf(load_f32<T>(s.q, c.wave * D + d), s.kn[d], sp);
      const float sv = wave_sum(sp) * sl2;
      const float mn = fmaxf(m, sv);
      const float alpha = __builtin_amdgcn_exp2f(m - mn);
      const float pr = __builtin_amdgcn_exp2f(sv - mn);
      if (c.lane == 0) {
        fin_a[c.wave] = alpha;
        fin_p[c.wave] = pr;
        fin_l[c.wave] = fmaf(l, alpha, pr);
      }
    }
    // partials of the position steps -> the kh == 0 wave of each dim block
    float* part = s.sc;  // free now: [KH - 1][NBK][64 lanes][4]
    if (KH > 1 && kh > 0) *(float4*)(part + (((kh - 1) * NBK + nbk) * 64 + c.lane) * 4) = make_float4(o[0], o[1], o[2], o[3]);
    bar();
    if (kh == 0) {
#pragma unroll
      for (int k = 1; k < KH; ++k) {
        const float4 q4 = *(const float4*)(part + (((k - 1) * NBK + nbk) * 64 + c.lane) * 4);
        o[0] += q4.x;
        o[1] += q4.y;
        o[2] += q4.z;
        o[3] += q4.w;
      }
      const int d = nbk * 16 + lr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int hh = 4 * lq + i;
        if (hh < G) store_f32<T>(xin, hh * D + d, fmaf(fin_p[hh], s.vn[d], o[i] * fin_a[hh]) / fin_l[hh]);
      }
    }
    bar();
  }

  // GQA attention of the block's KV group g for its G query heads over
  // ctx = cache_len + 1 positions: cached rows from K / V tiles in LDS (the
  // first tile was loaded during phase A), the current row from s.kn / s.vn.
  // Per tile, threads score one position against every head; then wave h
  // runs head h's online softmax over the tile and its P V (lane = dims).
  // The output, rounded to T, goes to xin (the o_proj input).
  __device__ __forceinline__ static void attention(const Ctx& c, int layer, int g, const AttnLds& s, T* xin,
                                                   int trs) {
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
        if (c.wave == 0) {
          tile_load(c, kc, vc, p0, np, s);
          wait_vm0();
        }
        bar();
      }
      // ---- scores of the tile
      if constexpr (EPW == 2) {
        // MFMA 16x16x16 (bf16 in, fp32 out): A = the q heads (rows, padded
        // to 16), B = 16 positions' keys; lane l holds A[l % 16][4 (l / 16) ..
        // + 3] and B[4 (l / 16) .. + 3][l % 16] of each 16-dim step, and gets
        // D[4 (l / 16) + i][l % 16]. Wave w scores position blocks w, w + 8, ...
        typedef short short4_t __attribute__((ext_vector_type(4)));
        typedef float float4_t __attribute__((ext_vector_type(4)));
        constexpr int KS = D / 16;
        const int lr = c.lane % 16, lq = c.lane / 16;
        short4_t qa[KS];
#pragma unroll
        for (int kb = 0; kb < KS; ++kb) {
          const uint2 v = lr < G ? *(const uint2*)(s.q + lr * D + kb * 16 + 4 * lq) : make_uint2(0, 0);
          qa[kb] = __builtin_bit_cast(short4_t, v);
        }
        for (int blk = c.wave; blk * 16 < np; blk += LWAVES) {
          const int r = blk * 16 + lr;
          const char* krow = s.kt + r * PPR * 16;
          float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kb = 0; kb < KS; ++kb) {
            const int piece = 2 * kb + (lq >> 1);
            const uint2 v =
                r < np ? *(const uint2*)(krow + ((piece ^ (r % PPR)) * 16) + (lq & 1) * 8) : make_uint2(0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(qa[kb], __builtin_bit_cast(short4_t, v), acc, 0, 0, 0);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int hh = 4 * lq + i;
            if (hh < G && r < np) s.sc[hh * TP + r] = acc[i] * p.scale;
          }
        }
      } else
      // thread = position, every head
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
      const float lt = fmaf(l, alpha, pr);
      if (pg == 0) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = fmaf(pr, s.vn[dc * 8 + e], acc[e] * alpha) / lt;
        if constexpr (EPW == 2) {
          *(uint4*)(xin + h * D + dc * 8) =
              make_uint4(pack_word<T>(o), pack_word<T>(o + 2), pack_word<T>(o + 4), pack_word<T>(o + 6));
        } else {
          *(float4*)(xin + h * D + dc * 8) = make_float4(o[0], o[1], o[2], o[3]);
          *(float4*)(xin + h * D + dc * 8 + 4) = make_float4(o[4], o[5], o[6], o[7]);
        }
      }
    }
    bar();
  }

  // ---------------------------------------------------------------- block glue
  // x += add (MODE 0: stage holds dtype words of the previous down; MODE 1:
  // stage holds the Hkv groups' fp32 o_proj partials, rounded to the dtype
  // once summed; MODE 2: nothing to add), each sum rounded to the dtype
  // (layer.py:63-64); then xin = dtype((x * rsqrt(mean(x^2) + eps)) * w) in
  // fp32 (layer.py:39-42), w being the norm weight in LDS. Thread t owns
  // elements 4t .. 4t + 3 (H <= 4 * LT, checked on the host).
  template <int MODE>
  __device__ __forceinline__ static void x_add_norm(const Ctx& c, float* xs, const uint64_t* stage, const T* w,
                                                    T* xin, float* red) {
    const int H = c.p->H;
    const int gi = c.tid;
    const bool in = gi < H / 4;
    float4* xs4 = (float4*)xs;
    float xv[4] = {0.f, 0.f, 0.f, 0.f};
    if (in) {
      const float4 v = xs4[gi];
      xv[0] = v.x;
      xv[1] = v.y;
      xv[2] = v.z;
      xv[3] = v.w;
      if constexpr (MODE == 0) {
        const uint4* st4 = (const uint4*)stage;
        float ad[4];
        if constexpr (EPW == 2) {  // words 2 gi, 2 gi + 1
          const uint4 a = st4[gi];
          ad[0] = word_elem<T>(a.x, 0);
          ad[1] = word_elem<T>(a.x, 1);
          ad[2] = word_elem<T>(a.z, 0);
          ad[3] = word_elem<T>(a.z, 1);
        } else {
          const uint4 a = st4[2 * gi], b = st4[2 * gi + 1];
          ad[0] = __uint_as_float(a.x);
          ad[1] = __uint_as_float(a.z);
          ad[2] = __uint_as_float(b.x);
          ad[3] = __uint_as_float(b.z);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = round_to<T>(add_rn(xv[e], ad[e]));
      } else if constexpr (MODE == 1) {
        float ad[4] = {0.f, 0.f, 0.f, 0.f};
        for (int g = 0; g < c.p->Hkv; ++g) {
          const uint4* st4 = (const uint4*)(stage + (int64_t)g * H);
          const uint4 a = st4[2 * gi], b = st4[2 * gi + 1];
          ad[0] += __uint_as_float(a.x);
          ad[1] += __uint_as_float(a.z);
          ad[2] += __uint_as_float(b.x);
          ad[3] += __uint_as_float(b.z);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = round_to<T>(add_rn(xv[e], round_to<T>(ad[e])));
      }
      if constexpr (MODE != 2) xs4[gi] = make_float4(xv[0], xv[1], xv[2], xv[3]);
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) ss = add_rn(ss, mul_rn(xv[e], xv[e]));
    ss = wave_sum(ss);
    if (c.lane == 0) red[c.wave] = ss;
    bar();
    float tot = 0.f;
#pragma unroll
    for (int k = 0; k < LWAVES; ++k) tot = add_rn(tot, red[k]);
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(add_rn(__fdiv_rn(tot, (float)H), c.p->eps)));
    if (in) {
      float wv[4], o[4];
      if constexpr (EPW == 2) {
        const uint2 a = ((const uint2*)w)[gi];
        wv[0] = word_elem<T>(a.x, 0);
        wv[1] = word_elem<T>(a.x, 1);
        wv[2] = word_elem<T>(a.y, 0);
        wv[3] = word_elem<T>(a.y, 1);
      } else {
        const float4 a = ((const float4*)w)[gi];
        wv[0] = a.x;
        wv[1] = a.y;
        wv[2] = a.z;
        wv[3] = a.w;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = mul_rn(mul_rn(xv[e], r), wv[e]);
      if constexpr (EPW == 2) {
        ((uint2*)xin)[gi] = make_uint2(pack_word<T>(o), pack_word<T>(o + 2));
      } else {
        ((float4*)xin)[gi] = make_float4(o[0], o[1], o[2], o[3]);
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
    T* nws = (T*)(lds + p.lds_norm);  // the current RMSNorm weight
    float* red = (float*)(lds + p.lds_misc);
    float* amv = red + LWAVES;
    int64_t* ami = (int64_t*)(lds + p.lds_misc + 64 * 4);
    AttnLds at;  // K / V tiles in their own region; the rest aliases stage (free in phase B)
    at.kt = lds + p.lds_tile;
    at.vt = at.kt + TP * PPR * 16;
    at.q = (T*)(lds + p.lds_stage);
    at.kn = (float*)(at.q + GMAXL * D);
    at.vn = at.kn + D;
    at.sc = at.vn + D;
    at.st = at.sc + GMAXL * TP;
    const int H = p.H, Hq = p.Hq, Hkv = p.Hkv, G = p.G;
    const uint4* xin4 = (const uint4*)xin;

    const bool w0 = c.wave == 0;  // wave 0 waits on the hand-offs; waves 1.. stream weights
    const int rw = c.wave - 1, nrw = NCW;
    float* rw_res = rowres + (w0 ? 0 : rw) * RPW;  // this weight wave's row results (phases A, C)

    const int npb = a_pairs_block(c);
    const int a_my_n = w0 ? 0 : a_my(npb, rw, nrw);
    int bg, br0, br1;
    b_rows_range(c, bg, br0, br1);
    const bool b_work = br1 > br0;
    const int bn = b_work ? br1 - br0 : 0;
    int cu0, cu1, du0, du1, lr0, lr1;
    c_range(c, cu0, cu1);
    d_range(c, du0, du1);
    lm_range(c, lr0, lr1);
    const int c_my = w0 ? 0 : (rw < cu1 - cu0 ? (cu1 - cu0 - 1 - rw) / nrw + 1 : 0);
    const int d_rows_n = EPW * (du1 - du0);
    const int64_t pos = p.positions[0];
    const bool pos_ok = pos >= 0 && pos < p.max_pos;
    // wave 0: the first K / V tile of a layer's attention (rows below
    // cache_len were written by earlier steps)
    auto tile_first = [&](int layer) {
      const int64_t lay_kv = (int64_t)layer * Hkv * p.S * D + (int64_t)bg * p.S * D;
      const int np0 = (int)(p.cache_len < TP ? p.cache_len : TP);
      tile_load(c, (const T*)p.k_cache + lay_kv, (const T*)p.v_cache + lay_kv, 0, np0, at);
    };

    // register batches: the next layer's rows of every phase
    uint4 bufA[JA * SA], bufB[JB * SB], bufC[JC * SC], bufD[JD * SD];
    // The gate/up and down batches go out in three parts each, after the
    // stores of three different phases, so that the loads of a phase's
    // weights are not one burst.
    constexpr int NC = JC * SC, ND = JD * SD;
#define ISSUE_C(K, W, LIVE) \
  rows_issue_part<JC, SC, NC*(K) / 3, NC*((K) + 1) / 3>(bufC, c_q(c, W, c_my, LIVE), rc, 0, 0, c.lane)
#define ISSUE_D(K, W, LIVE) \
  rows_issue_part<JD, SD, ND*(K) / 3, ND*((K) + 1) / 3>(bufD, d_q(c, W, d_rows_n, rw, nrw, LIVE), rd, 0, 0, c.lane)
    const auto ra = a_rows(c, rw, nrw);
    const auto rb = b_rows(c, br0, rw, nrw);
    const auto rc = c_rows(c, cu0, rw, nrw);
    const auto rd = d_rows(c, du0, rw, nrw);
    // lane 2 t + k: the k-th bias of the wave's t-th pair (loaded with the
    // layer's QKV rows) and its RoPE cos / sin (the same for every layer)
    float biasv = 0.f, cosv = 0.f, sinv = 0.f;
    const int a_lane_t = c.lane >> 1, a_lane_k = c.lane & 1;
    auto issue_bias = [&](const LoopLayerW& w, bool live) {
      if (!w0) {
        int hd, i;
        a_pair(c, rw, nrw, a_lane_t, hd, i);
        const bool in = live && a_lane_t < a_my_n;
        const int k = in ? hd * D + i + a_lane_k * HALF : 0;
        if constexpr (EPW == 2) {
          typedef __attribute__((address_space(1))) const uint16_t gU16;
          biasv = bf16_to_f32(((const gU16*)w.bqkv)[k]);
        } else {
          typedef __attribute__((address_space(1))) const float gF;
          biasv = ((const gF*)w.bqkv)[k];
        }
      }
    };
    if (!w0) {
      int hd, i;
      a_pair(c, rw, nrw, a_lane_t, hd, i);
      if (pos_ok && a_lane_t < a_my_n && hd < Hq + Hkv) {
        typedef __attribute__((address_space(1))) const float gF;
        cosv = ((const gF*)p.cos_tab)[pos * D + i + a_lane_k * HALF];
        sinv = ((const gF*)p.sin_tab)[pos * D + i + a_lane_k * HALF];
      }
      const LoopLayerW& l0 = p.layers[0];
      rows_issue<JA, SA>(bufA, a_q(c, l0, a_my_n, true), ra, 0, 0, c.lane);
      issue_bias(l0, true);
      rows_issue<JB, SB>(bufB, b_q(c, l0, bg, bn, rw, nrw, true), rb, 0, 0, c.lane);
      ISSUE_C(0, l0, true);
      ISSUE_C(1, l0, true);
      ISSUE_D(0, l0, true);
    } else {
      // embedding (embedding.py:44-46): every block gathers the row
      const int64_t id = p.ids[0];
      const bool ok = id >= 0 && id < p.V;
      const T* row = (const T*)p.embed + (ok ? id : 0) * H;
      for (int i = c.lane; i < H; i += 64) xs[i] = ok ? load_f32<T>(row, i) : __builtin_nanf("");
      if (!pos_ok && c.b == 0 && c.lane == 0)
        __hip_atomic_fetch_or(&p.ctrl[LOOP_CTRL_ERROR], (uint32_t)LOOP_ERR_POSITION, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
    }
    c.mark(LOOP_TR_START);
    if (p.trace && c.tid == 0)
      p.trace[((int64_t)c.b * p.trace_slots + 1 + p.L * LOOP_TR_PER_LAYER + 3) * LWAVES + 1] = clock64();

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

      // ======== A: x += down (previous layer), RMSNorm, QKV + bias + RoPE ========
      if (w0) {
        lds_fetch(c, lw.ln1, H * (int)sizeof(T), nws);
        if (b_work) tile_first(layer);  // this layer's first K / V tile, ahead of phase B
        if (layer > 0)
          ll_gather(c, p.ll + (int64_t)(layer - 1) * p.ll_layer_words + p.off_down, H / EPW, stage);
        else
          wait_vm0();
        c.mark(tr + LOOP_TR_A_ISSUED);  // wave 0: the hand-off arrived
      }
      bar();
      if (layer > 0)
        x_add_norm<0>(c, xs, stage, nws, xin, red);
      else
        x_add_norm<2>(c, xs, stage, nws, xin, red);
      c.mark(tr + LOOP_TR_A_IN);
      if (!w0) {
        rows_consume<T, JA, SA>(bufA, a_q(c, lw, a_my_n, true), ra, xin4, c.lane, [&](int s, float v) {
          if (c.lane == 0) rw_res[s] = v;
        });
        const float bias_now = biasv;
        wave_lds_fence();
        // lane t: the wave's t-th pair
        const float b0 = __shfl(bias_now, 2 * a_lane_t), b1 = __shfl(bias_now, 2 * a_lane_t + 1);
        const float cs0 = __shfl(cosv, 2 * a_lane_t), cs1 = __shfl(cosv, 2 * a_lane_t + 1);
        const float sn0 = __shfl(sinv, 2 * a_lane_t), sn1 = __shfl(sinv, 2 * a_lane_t + 1);
        if (c.lane < a_my_n) {
          const int t = c.lane;
          int hd, i;
          a_pair(c, rw, nrw, t, hd, i);
          // F.linear output with bias, rounded to the dtype (fused.py:58)
          const float va = round_to<T>(add_rn(rw_res[2 * t], b0));
          const float vb = round_to<T>(add_rn(rw_res[2 * t + 1], b1));
          float o[2] = {va, vb};
          if (hd < Hq + Hkv) {
            // rotate: x * cos + rotate_half(x) * sin, fp32, each op rounded,
            // then cast (rope.py:57-62)
            if (pos_ok) {
              o[0] = round_to<T>(add_rn(mul_rn(va, cs0), -mul_rn(vb, sn0)));
              o[1] = round_to<T>(add_rn(mul_rn(vb, cs1), mul_rn(va, sn1)));
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
        c.mark(tr + LOOP_TR_A_ISSUED);  // weight waves: results stored
        // the next loads go out once this phase's results are on their way
        rows_issue<JA, SA>(bufA, a_q(c, nw, a_my_n, more), ra, 0, 0, c.lane);
        issue_bias(nw, more);
        ISSUE_C(2, lw, true);
        ISSUE_D(1, lw, true);
      }
      c.mark(tr + LOOP_TR_A_OUT);

      // ======== B: attention of group bg + its o_proj share for rows [br0, br1) ========
      if (b_work) {
        if (w0) {
          const int gw = (G + 2) * HALF * WPP;  // the group's q heads, k head, v head
          ll_gather(c, ll_qkv + (int64_t)bg * gw, gw, qstage);
          c.mark(tr + LOOP_TR_B_ISSUED);  // wave 0: the hand-off arrived
        }
        bar();
      }
      if (b_work) {
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
      }
      if (b_work) {
        if constexpr (EPW == 2)
          attention_mfma(c, layer, bg, at, xin, tr);
        else
          attention(c, layer, bg, at, xin, tr);
        c.mark(tr + LOOP_TR_B_ATTN);
      }
      if (!w0) {
        rows_consume<T, JB, SB>(bufB, b_q(c, lw, bg, bn, rw, nrw, true), rb, xin4, c.lane, [&](int s, float v) {
          if (c.lane == 0) ll_store(ll_p + (int64_t)bg * H + br0 + rw + nrw * s, c.epoch, __float_as_uint(v));
        });
        c.mark(tr + LOOP_TR_B_ISSUED);  // weight waves: results stored
        rows_issue<JB, SB>(bufB, b_q(c, nw, bg, bn, rw, nrw, more), rb, 0, 0, c.lane);
        ISSUE_D(2, lw, true);
      }
      c.mark(tr + LOOP_TR_B_OUT);

      // ======== C: x += dtype(o_proj), RMSNorm, gate/up, SwiGLU ========
      if (w0) {
        lds_fetch(c, lw.ln2, H * (int)sizeof(T), nws);
        ll_gather(c, ll_p, Hkv * H, stage);
        c.mark(tr + LOOP_TR_C_ISSUED);  // wave 0: the hand-off arrived
      }
      bar();
      x_add_norm<1>(c, xs, stage, nws, xin, red);
      c.mark(tr + LOOP_TR_C_IN);
      if (!w0) {
        rows_consume<T, JC, SC>(bufC, c_q(c, lw, c_my, true), rc, xin4, c.lane, [&](int s, float v) {
          if (c.lane == 0) rw_res[s] = v;
        });
        wave_lds_fence();
        if (c.lane < c_my) {  // lane t: the wave's t-th unit
          const int t = c.lane;
          float a[EPW];
#pragma unroll
          for (int e = 0; e < EPW; ++e)
            a[e] = swiglu<T>(round_to<T>(rw_res[2 * EPW * t + 2 * e]),
                             round_to<T>(rw_res[2 * EPW * t + 2 * e + 1]));  // mlp.py:38
          ll_store(ll_act + cu0 + rw + nrw * t, c.epoch, pack_word<T>(a));
        }
        c.mark(tr + LOOP_TR_C_ISSUED);  // weight waves: results stored
        ISSUE_C(0, nw, more);
      }
      c.mark(tr + LOOP_TR_C_OUT);

      // ======== D: down projection ========
      if (w0) {
        ll_gather(c, ll_act, p.I / EPW, stage);
        c.mark(tr + LOOP_TR_D_ISSUED);  // wave 0: the hand-off arrived
      }
      bar();
      {
        // payloads of word pairs -> xin (I / EPW is even: I and H are even)
        const uint4* st4 = (const uint4*)stage;
        uint2* x2 = (uint2*)xin;
        for (int i = c.tid; i < p.I / EPW / 2; i += LT) {
          const uint4 v = st4[i];
          x2[i] = make_uint2(v.x, v.z);
        }
      }
      bar();
      c.mark(tr + LOOP_TR_D_IN);
      if (!w0) {
        rows_consume<T, JD, SD>(bufD, d_q(c, lw, d_rows_n, rw, nrw, true), rd, xin4, c.lane, [&](int s, float v) {
          if (c.lane == 0) rowres[rw + nrw * s] = v;
        });
        c.mark(tr + LOOP_TR_D_ISSUED);  // weight waves: results in LDS
        ISSUE_C(1, nw, more);
        ISSUE_D(0, nw, more);
      }
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

#undef ISSUE_C
#undef ISSUE_D

    // ======== final norm, LM head, greedy pick ========
    {
      const int tr = 1 + p.L * LOOP_TR_PER_LAYER;
      uint4 bufL[JL * SL];
      if (!w0) rows_issue<JL, SL>(bufL, lm_q(c, lr1 - lr0), lm_rows(c, lr0), 0, 0, c.lane);
      if (w0) {
        lds_fetch(c, p.final_norm, H * (int)sizeof(T), nws);
        ll_gather(c, p.ll + (int64_t)(p.L - 1) * p.ll_layer_words + p.off_down, H / EPW, stage);
      }
      bar();
      c.mark(tr);
      x_add_norm<0>(c, xs, stage, nws, xin, red);
      if (!w0) {
        const int cw = c.cw;
        rows_consume<T, JL, SL>(bufL, lm_q(c, lr1 - lr0), lm_rows(c, lr0), xin4, c.lane, [&](int s, float v) {
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
      if (c.b == 0 && w0) {
        ll_gather(c, part, 2 * c.nb, stage);
        float v = -__builtin_inff();
        int64_t i = INT64_MAX;
        for (int k = c.lane; k < c.nb; k += 64) {
          const float vk = __uint_as_float(payload(stage[2 * k]));
          const int64_t ik = (int64_t)payload(stage[2 * k + 1]);
          if (argmax_better(vk, ik, v, i)) {
            v = vk;
            i = ik;
          }
        }
        wave_argmax(v, i);
        if (c.lane == 0) {
          if (p.next_tok) p.next_tok[0] = i;
          p.ctrl[LOOP_CTRL_EPOCH] = c.epoch;
        }
        c.mark(tr + 2);
        if (p.trace && c.lane == 0) p.trace[((int64_t)c.b * p.trace_slots + tr + 3) * LWAVES + 2] = clock64();
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
}

inline int align_up(int v, int a) { return (v + a - 1) / a * a; }

}  // namespace

const void* loop_kernel(int dtype, int D) {
  return dtype == MINITP_F32 ? pick_kernel<float>(D) : pick_kernel<bf16>(D);
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
  const int attn_bytes = GMAXL * D * es + 2 * D * 4 + GMAXL * tp * 4 + 4 * GMAXL * 4;
  // gathered hand-off words (8 bytes each, whole 128-word copies)
  const int epw_ = es == 4 ? 1 : 2;
  const int gmax = std::max(std::max(c.kv_heads * c.hidden, c.hidden / epw_), std::max(c.intermediate / epw_, 2 * nb));
  if (gmax > 64 * 128) return "a hand-off exceeds 8192 words";
  const int stage_words = align_up(gmax, 128);
  L.stage = take(std::max(attn_bytes, stage_words * 8));
  L.qstage = take(align_up((G + 2) * (D / 2) * (2 / epw_), 128) * 8);
  // row results: per weight wave (phases A and C), the block's down rows,
  // the block's LM-head rows
  const int npa = (c.heads + 2 * c.kv_heads) * (D / 2);
  const int epw = es == 4 ? 1 : 2;
  const int rows_d = epw * ((c.hidden / epw + nb - 1) / nb);
  const int rows_lm = (c.vocab + nb - 1) / nb;
  L.rowres = take(std::max(std::max(NCW * LOOP_ROWS_PER_WAVE, rows_d), rows_lm) * 4 + 16);
  L.norm = take(align_up(c.hidden * es, 1024));
  L.misc = take(64 * 4 + LWAVES * 8);
  if ((npa + nb - 1) / nb > 64) return "more than 64 QKV pairs per block";
  if (c.hidden > 4 * LOOP_THREADS) return "hidden size above 2048";
  {
    const int upb = (c.intermediate / epw + nb - 1) / nb;  // gate/up units per block
    if (2 * epw * ((upb + NCW - 1) / NCW) > LOOP_ROWS_PER_WAVE) return "too many gate/up rows per wave";
  }
  L.bytes = off;
  if (L.bytes > 160 * 1024) return "LDS layout exceeds 160 KiB";
  if (out) *out = L;
  return nullptr;
}

}  // namespace minitp
