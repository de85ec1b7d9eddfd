// Large bf16 linear layers of a prompt on gfx950's 32x32x16 MFMA:
// y[M, N] = bf16(x[M, K] W[N, K]^T (+ bias)), or with the SwiGLU pairing of a
// [gate; up] weight, act[M, I] = bf16(bf16(silu(g)) * u) where g, u are the
// bf16-rounded products with rows j and I + j of W (mlp.py:34-38,
// fused.py:102-104; F.linear semantics of fused.py:57-61 / linear.py:117).
//
// Block tile 256 x 256 x (K steps of 64), 1,024 threads = 16 waves in a
// 4 x 4 grid (four per SIMD), each wave owning a 64 x 64 output tile as 2 x 2
// fragments of 32 x 32 (16 fp32 accumulators per lane each). Both operands
// are K-contiguous (x rows, W rows), the layout the MFMA operands want:
//   v_mfma_f32_32x32x16_bf16: lane l holds A[l % 32][8 (l / 32) + 0..7] and
//   B[8 (l / 32) + 0..7][l % 32]; accumulator register r of lane l is
//   D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
// K steps are staged in LDS (two buffers, 64 KiB each: 256 rows of x and of
// W, 128 bytes per row), each 16-byte chunk c of row r stored at chunk
// position c ^ ((r / 2) & 7), so the lanes reading one fragment column spread
// over all banks. The operands go from global memory straight into LDS
// (gfx950's buffer_load_dwordx4 ... lds: no registers, no LDS write
// instructions), the next step's while a step's MFMAs run, one barrier per
// step. Loads are buffer loads: rows past M or N read zeros, so no load is
// predicated.
//
// Measured at the 7B prefill shapes (16,384 rows): against 8 waves of
// 128 x 64 with register staging, gate/up 3.86 -> 3.67 ms, QKV 0.48 -> 0.46,
// down unchanged (1.91); the matrix pipes are then busy 71 % of the cycles at
// the clock the part holds (1.63 GHz; 72 % with the operand loads left out,
// at 1.81 GHz). Slower: the same 8-wave layout with DMA staging (no faster),
// plus an L2 prefetch of the step after next split over the blocks sharing a
// panel (5-8 % slower), 4 waves of 128 x 128 (20 % slower), 16 waves with
// register staging (gate/up 6.8 ms).
//
// Tile order: blocks are dispatched to the 8 XCDs round-robin (block b runs on
// XCD b % 8, each XCD with its own L2). Block b takes tile (b % 8) * per_xcd +
// b / 8, so each XCD works through one contiguous range of tiles, and inside
// a range tiles go in groups of 8 row-tiles (all column tiles of one group of
// x rows before the next): the 32 blocks an XCD runs at once share 8 x panels
// and 4 W panels through its L2.
//
// Deterministic: every output element is one fixed-order fp32 sum over K.
#include "common.h"
#include "kernels.h"

namespace minitp {

namespace {

typedef __bf16 bf16x8_g __attribute__((ext_vector_type(8)));
typedef float f32x16_g __attribute__((ext_vector_type(16)));

constexpr int TM = 256, TN = 256, TK = 64;
constexpr int ROWB = TK * 2;  // bytes per row per stage
constexpr int A_BYTES = TM * ROWB, B_BYTES = TN * ROWB;
constexpr int STAGE_BYTES = A_BYTES + B_BYTES;  // 64 KiB
constexpr int LDS_TILE_BYTES = 2 * STAGE_BYTES;
constexpr int GROUP_M = 8;  // row tiles per group (4 measured the same, 16 and 32 slower)
// waves along N and M: 4 x 4 (64 x 64 wave tiles, four waves per SIMD; the
// default), 4 x 2 (128 x 64, two per SIMD) or 2 x 2 (128 x 128, one per SIMD)
#ifndef MINITP_TILE_WAVES_N
#define MINITP_TILE_WAVES_N 4
#endif
#ifndef MINITP_TILE_WAVES_M
#define MINITP_TILE_WAVES_M 4
#endif

// A row past the matrix: its voffset, plus any K offset in soffset, stays
// past the resource's range (operands are below DMA_OOB bytes and K below
// 2^27), so the load writes zeros.
constexpr uint32_t DMA_OOB = 0xF0000000u;

// Words of a raw buffer resource over [base, base + bytes) (SGPRs).
__device__ __forceinline__ u32x4 rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  u32x4 r;
  r.x = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)p);
  r.y = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));  // stride 0
  r.z = (uint32_t)__builtin_amdgcn_readfirstlane(bytes);
  r.w = 0x00020000u;
  return r;
}

// 16 bytes per lane from the resource at voff + soff into LDS: lane l's
// bytes land at LDS byte address lds_addr + 16 l (lds_addr wave-uniform, in
// m0); an offset past the range writes zeros. Issued as asm so that the
// compiler does not make every later LDS read wait for these loads: the
// kernel waits for them itself (vmcnt(0) before the barrier that publishes
// the stage).
__device__ __forceinline__ void dma16(u32x4 r, uint32_t voff, uint32_t soff, uint32_t lds_addr) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(lds_addr) : "memory");
}

// byte offset of chunk c of row r inside an operand's stage buffer. The LDS
// has 64 banks of 4 bytes (256 bytes across), and a ds_read_b128 serves 16
// lanes at a time: the 16 lanes of a fragment read (rows r .. r + 15, one
// chunk column) fall on 16 distinct 16-byte slots when row pairs (2i, 2i + 1)
// take chunk positions c ^ i.
#ifndef MINITP_TILE_SWZ_SHIFT
#define MINITP_TILE_SWZ_SHIFT 1
#endif
__device__ __forceinline__ int lds_off(int r, int c) {
  return r * ROWB + ((c ^ ((r >> MINITP_TILE_SWZ_SHIFT) & 7)) << 4);
}

enum { TILE_STORE = 0, TILE_SWIGLU = 1 };

template <int EPI, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_tile_kernel(const bf16* __restrict__ x, int64_t ldx,
                                                             const bf16* __restrict__ w, const bf16* __restrict__ bias,
                                                             bf16* __restrict__ y, int64_t ldy, int M, int N, int K,
                                                             int tiles_m, int tiles_n, int per_xcd, int full_tiles,
                                                             int tail_split, float* __restrict__ tail_part,
                                                             uint32_t* __restrict__ tail_cnt) {
  constexpr int TTHREADS = 64 * WAVES_M * WAVES_N;
  constexpr int WTM = TM / WAVES_M, FM = WTM / 32;  // wave tile rows
  constexpr int WTN = TN / WAVES_N, FN = WTN / 32;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int b = blockIdx.x;
  // blocks [0, 8 per_xcd): tiles [0, full_tiles), one each, in
  // XCD-contiguous ranges; past that (the split last round, where
  // 8 per_xcd == full_tiles) tail_split blocks per remaining tile, block part
  // p taking the p-th share of the K steps
  const bool split_blk = b >= 8 * per_xcd;
  int t, part = 0;
  if (!split_blk) {
    const int local = b >> 3;
    t = (b & 7) * per_xcd + local;
    if (t >= full_tiles) return;
  } else {
    t = full_tiles + (b - 8 * per_xcd) / tail_split;
    part = (b - 8 * per_xcd) % tail_split;
    if (t >= tiles_m * tiles_n) return;
  }
  const int group = t / (GROUP_M * tiles_n);
  const int first_m = group * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  const int in_group = t - group * GROUP_M * tiles_n;
  const int tm = first_m + in_group % gsz, tn = in_group / gsz;
  const int m0 = tm * TM;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  // Rows of W this block streams: STORE, tile columns n0 .. n0 + 255; SWIGLU,
  // per 64-row group g of the tile, 32 gate rows then the 32 matching up rows
  // (output columns c0 + 32 g .. + 31, c0 = 128 tn), so a wave's two column
  // fragments are a gate fragment and its up fragment.
  auto w_row = [&](int r) -> int {
    if (EPI == TILE_SWIGLU) {
      const int g = r >> 6, within = r & 63, col = tn * 128 + g * 32 + (within & 31);
      if (col >= N) return -1;
      return within < 32 ? col : N + col;
    }
    const int n = tn * TN + r;
    return n < N ? n : -1;
  };

  const int64_t w_rows = EPI == TILE_SWIGLU ? 2LL * N : (int64_t)N;

  f32x16_g acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // fragment rows this lane reads
  const int ar0 = wm * WTM + (lane & 31), br0 = wn * WTN + (lane & 31);
  const int half = lane >> 5;

  // A stage is 64 pieces of 1 KiB, each 8 rows x 128 bytes of one operand
  // (x rows 0..255, then W rows), in lds_off's layout: lane l of the wave
  // moving a piece takes the row's chunk whose swizzled position is l % 8, so
  // the piece lands as one contiguous KiB. Wave w moves pieces w PPW ..
  // w PPW + PPW - 1 of every stage.
  constexpr int NWAVES = WAVES_M * WAVES_N, PIECES = (TM + TN) / 8, PPW = PIECES / NWAVES;
  static_assert(PIECES % NWAVES == 0 && TM % 8 == 0, "pieces must split evenly over the waves");
  const int wv = __builtin_amdgcn_readfirstlane(wave);  // uniform: the pieces' operand and LDS address
  const u32x4 xq = rsrc_words(x, (uint32_t)(((int64_t)(M - 1) * ldx + K) * 2));
  const u32x4 wq = rsrc_words(w, (uint32_t)(w_rows * K * 2));
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  uint32_t voff[PPW];  // byte offset of the lane's chunk at k = 0 (DMA_OOB: a row past the matrix)
  int kc[PPW];         // its first k
#pragma unroll
  for (int j = 0; j < PPW; ++j) {
    const int p = wv * PPW + j, is_w = p >= TM / 8;
    const int r = 8 * (is_w ? p - TM / 8 : p) + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> MINITP_TILE_SWZ_SHIFT) & 7);
    kc[j] = c * 8;
    if (!is_w) {
      voff[j] = m0 + r < M ? (uint32_t)(((int64_t)(m0 + r) * ldx + c * 8) * 2) : DMA_OOB;
    } else {
      const int wrow = w_row(r);
      voff[j] = wrow >= 0 ? (uint32_t)(((int64_t)wrow * K + c * 8) * 2) : DMA_OOB;
    }
  }
  auto issue = [&](int kstep, int stage) {
    const int k0 = kstep * TK;
    const uint32_t base = lds0 + stage * STAGE_BYTES;
    if (k0 + TK <= K) {
      const uint32_t so = (uint32_t)__builtin_amdgcn_readfirstlane(k0 * 2);
#pragma unroll
      for (int j = 0; j < PPW; ++j) {
        const int p = wv * PPW + j;
        dma16(p >= TM / 8 ? wq : xq, voff[j], so, (uint32_t)__builtin_amdgcn_readfirstlane(base + p * 1024));
      }
    } else {
      // the K tail: chunks at or past K read zeros
#pragma unroll
      for (int j = 0; j < PPW; ++j) {
        const int p = wv * PPW + j;
        const uint32_t v = voff[j] != DMA_OOB && k0 + kc[j] < K ? voff[j] + (uint32_t)k0 * 2 : DMA_OOB;
        dma16(p >= TM / 8 ? wq : xq, v, 0u, (uint32_t)__builtin_amdgcn_readfirstlane(base + p * 1024));
      }
    }
  };

  // K step kt: the MFMAs read stage kt % 2 while the pieces of step kt + 1
  // load into the other stage; fragment reads run one 16-wide substep ahead
  // of the MFMAs that use them (two register sets); one barrier per step.
  const int nk_all = (K + TK - 1) / TK;
  const int kper = (nk_all + tail_split - 1) / tail_split;
  const int kb = split_blk ? part * kper : 0;
  const int nk = split_blk ? min(nk_all, kb + kper) - kb : nk_all;  // steps of this block
  constexpr int KS = TK / 16;                                       // MFMA k substeps per step
  issue(kb, 0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    // the next step's pieces go to the other stage, which every wave
    // finished reading before the barrier that ended the previous step
    if (kt + 1 < nk) issue(kb + kt + 1, (kt + 1) & 1);
    const char* sa = lds + (kt & 1) * STAGE_BYTES;
    const char* sb = sa + A_BYTES;
    bf16x8_g av[2][FM], bv[2][FN];
    auto fetch = [&](int ks, bf16x8_g(&a)[FM], bf16x8_g(&bb)[FN]) {
      const int c = ks * 2 + half;
#pragma unroll
      for (int i = 0; i < FM; ++i) a[i] = *(const bf16x8_g*)(sa + lds_off(ar0 + i * 32, c));
#pragma unroll
      for (int j = 0; j < FN; ++j) bb[j] = *(const bf16x8_g*)(sb + lds_off(br0 + j * 32, c));
    };
    fetch(0, av[0], bv[0]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) fetch(ks + 1, av[(ks + 1) & 1], bv[(ks + 1) & 1]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[ks & 1][i], bv[ks & 1][j], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // this wave's pieces of step kt + 1 are in LDS
    __syncthreads();
  }

  // ---- the split last round: partials, the last block adds them ----------
  // Each block stores its fp32 tile device-coherent ([register quad][thread]
  // 16-byte pieces: a wave's stores are 1 KiB contiguous), waits for their
  // completion, and counts itself in on the tile's arrival word; the block
  // that brings the word to tail_split adds the parts in part order (the
  // same bits whatever the arrival order), resets the word and runs the
  // epilogue. Sums over K come out in two or more runs instead of one: a
  // different but equally fixed order.
  if (split_blk) {
    __shared__ int last_blk;
    constexpr int QUADS = FM * FN * 4;
    const int slot = t - full_tiles;
    const __amdgpu_buffer_rsrc_t pr =
        span_rsrc(tail_part, (uint32_t)((int64_t)(slot + 1) * tail_split * QUADS * TTHREADS * 16));
    auto poff = [&](int p, int qd) -> uint32_t {
      return (uint32_t)(((((int64_t)slot * tail_split + p) * QUADS + qd) * TTHREADS + tid) * 16);
    };
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const u32x4 v = {__float_as_uint(acc[i][j][4 * r4]), __float_as_uint(acc[i][j][4 * r4 + 1]),
                           __float_as_uint(acc[i][j][4 * r4 + 2]), __float_as_uint(acc[i][j][4 * r4 + 3])};
          __builtin_amdgcn_raw_buffer_store_b128(v, pr, poff(part, (i * FN + j) * 4 + r4), 0, 16 /* sc1 */);
        }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the partials are out
    __syncthreads();
    if (tid == 0) {
      const uint32_t old = __hip_atomic_fetch_add(tail_cnt + slot, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_blk = old == (uint32_t)(tail_split - 1);
      if (last_blk) __hip_atomic_store(tail_cnt + slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last_blk) return;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          float v[4] = {0.f, 0.f, 0.f, 0.f};
          for (int p = 0; p < tail_split; ++p) {
            float x4[4];
            if (p == part) {
#pragma unroll
              for (int e = 0; e < 4; ++e) x4[e] = acc[i][j][4 * r4 + e];
            } else {
              const u32x4 w4 = __builtin_bit_cast(
                  u32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, poff(p, (i * FN + j) * 4 + r4), 0, 16 /* sc1 */));
              x4[0] = __uint_as_float(w4.x);
              x4[1] = __uint_as_float(w4.y);
              x4[2] = __uint_as_float(w4.z);
              x4[3] = __uint_as_float(w4.w);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = p == 0 ? x4[e] : v[e] + x4[e];
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][j][4 * r4 + e] = v[e];
        }
  }

  // epilogue: lane holds column (lane % 32) of rows 8 (r / 4) + 4 half + r % 4
  const int row_base = m0 + wm * WTM + 4 * half;
  if (EPI == TILE_SWIGLU) {
    // column fragments 2p (gate) and 2p + 1 (up) of 64-row group wn (WTN / 64) + p
#pragma unroll
    for (int pr = 0; pr < FN / 2; ++pr) {
      const int col = tn * 128 + (wn * (WTN / 64) + pr) * 32 + (lane & 31);
      if (col >= N) continue;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = row_base + i * 32 + 8 * (r >> 2) + (r & 3);
          if (row < M) {
            const float g = round_to<bf16>(acc[i][2 * pr][r]), u = round_to<bf16>(acc[i][2 * pr + 1][r]);
            y[(int64_t)row * ldy + col].bits = f32_to_bf16(swiglu<bf16>(g, u));
          }
        }
    }
  } else {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = tn * TN + wn * WTN + j * 32 + (lane & 31);
      if (col >= N) continue;
      const float bv = bias != nullptr ? bf16_to_f32(bias[col].bits) : 0.f;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = row_base + i * 32 + 8 * (r >> 2) + (r & 3);
          if (row < M) y[(int64_t)row * ldy + col].bits = f32_to_bf16(acc[i][j][r] + bv);
        }
    }
  }
}

// CUs of the current device (the tile rounds' width)
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

// K steps each part of a tile split over K runs at least (so that the
// pipeline fills and the fp32 partials stay small against the work)
constexpr int SPLIT_MIN_STEPS = 16;
// at most this many parts (7B down projection at 512 tokens, TTFT: 4 or 6
// parts 12.43-12.55 ms, 8 parts 12.63-12.66 ms, the split-K GEMM 12.82-12.84)
#ifndef MINITP_TILE_SPLIT_MAX
#define MINITP_TILE_SPLIT_MAX 4
#endif

template <int EPI>
int launch_tile(hipStream_t st, const void* x, int64_t ldx, const void* w, const void* bias, void* y, int64_t ldy,
                int64_t M, int64_t N, int64_t K, TileTail tail, bool split_all = false) {
  constexpr int WM = MINITP_TILE_WAVES_M, WN = MINITP_TILE_WAVES_N;
  constexpr int64_t PART_BYTES = (int64_t)TM * TN * 4;  // one fp32 tile
  const void* kern = (const void*)gemm_tile_kernel<EPI, WM, WN>;
  if (const int rc = ensure_lds_limit(kern, LDS_TILE_BYTES)) return rc;
  const int tiles_m = (int)cdiv(M, TM);
  const int tiles_n = (int)cdiv(N, EPI == TILE_SWIGLU ? TN / 2 : TN);
  const int tiles = tiles_m * tiles_n;
  // One block per CU at a time (128 KiB of LDS): tiles run in rounds of
  // `cus`. A last round at most half full is split over K into S parts
  // (S rem <= cus blocks), so that it takes about 1/S of a round; it needs
  // the workspace and S <= the K steps.
  const int cus = device_cus();
  const int rem = tiles % cus, nk = (int)cdiv(K, TK);
  int split = 1;
  if (split_all) {
    // fewer tiles than half the CUs: every tile split over K
    split = std::min(std::min(cus / tiles, MINITP_TILE_SPLIT_MAX), nk / SPLIT_MIN_STEPS);
    while (split > 1 && (int64_t)tiles * split * PART_BYTES > TILE_TAIL_BYTES) --split;
    if (split < 2 || tiles > SPLIT_MAX_TUPLES || tail.part == nullptr || tail.count == nullptr) {
      set_error("gemm_tile: %d tiles of %d K steps do not split", tiles, nk);
      return MINITP_ERR_UNSUPPORTED;
    }
  } else if (tail.part != nullptr && tail.count != nullptr && tiles >= cus && rem > 0 && 2 * rem <= cus) {
    split = std::min(std::min(cus / rem, 4), nk);
    if ((int64_t)rem * split * PART_BYTES > TILE_TAIL_BYTES || rem > SPLIT_MAX_TUPLES) split = 1;
  }
  const int full = split_all ? 0 : split > 1 ? tiles - rem : tiles;
  const int per_xcd = (full + 7) / 8;
  const int grid = split_all ? tiles * split : 8 * per_xcd + (split > 1 ? rem * split : 0);
  hipLaunchKernelGGL((gemm_tile_kernel<EPI, WM, WN>), dim3((unsigned)grid), dim3(64 * WM * WN), LDS_TILE_BYTES, st,
                     (const bf16*)x, ldx, (const bf16*)w, (const bf16*)bias, (bf16*)y, ldy, (int)M, (int)N, (int)K,
                     tiles_m, tiles_n, per_xcd, full, split, tail.part, tail.count);
  MINITP_LAUNCH_CHECK();
  return MINITP_OK;
}

}  // namespace

// Whole rows of tiles (M a multiple of 256) but fewer tiles than half the
// CUs, and K long enough for two parts of SPLIT_MIN_STEPS: every tile split
// over K, its parts added by the tile's last block (the split-last-round
// machinery applied to all tiles).
bool gemm_tile_split_supported(int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy, bool swiglu) {
  const int64_t w_rows = swiglu ? 2 * N : N;
  const int64_t tiles = cdiv(M, TM) * cdiv(N, swiglu ? TN / 2 : TN);
  return M >= TM && M % TM == 0 && 2 * tiles <= device_cus() && cdiv(K, TK) >= 2 * SPLIT_MIN_STEPS && K % 8 == 0 &&
         ldx % 8 == 0 && ldx >= K && ldy >= N && M < (1LL << 31) && N < (1LL << 30) &&
         ((M - 1) * ldx + K) * 2 < DMA_OOB && w_rows * K * 2 < DMA_OOB && K < (1LL << 27);
}

int launch_gemm_tile_split(hipStream_t st, const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                           int64_t ldy, int64_t M, int64_t N, int64_t K, bool swiglu, TileTail tail) {
  if (!gemm_tile_split_supported(M, N, K, ldx, ldy, swiglu) || !aligned16(x) || !aligned16(w)) {
    set_error("gemm_tile: split shape M=%lld N=%lld K=%lld not served", (long long)M, (long long)N, (long long)K);
    return MINITP_ERR_UNSUPPORTED;
  }
  if (swiglu) return launch_tile<TILE_SWIGLU>(st, x, ldx, w, nullptr, y, ldy, M, N, K, tail, true);
  return launch_tile<TILE_STORE>(st, x, ldx, w, bias, y, ldy, M, N, K, tail, true);
}

bool gemm_tile_supported(int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy, bool swiglu) {
  const int64_t w_rows = swiglu ? 2 * N : N;
  const int64_t tiles = cdiv(M, TM) * cdiv(N, swiglu ? TN / 2 : TN);
  return M >= TM && tiles >= 96 && K % 8 == 0 && ldx % 8 == 0 && ldx >= K && ldy >= N && M < (1LL << 31) &&
         N < (1LL << 30) && ((M - 1) * ldx + K) * 2 < DMA_OOB && w_rows * K * 2 < DMA_OOB && K < (1LL << 27);
}

int launch_gemm_tile(hipStream_t st, const void* x, int64_t ldx, const void* w, const void* bias, void* y, int64_t ldy,
                     int64_t M, int64_t N, int64_t K, bool swiglu, TileTail tail) {
  if (!gemm_tile_supported(M, N, K, ldx, ldy, swiglu) || !aligned16(x) || !aligned16(w)) {
    set_error("gemm_tile: shape M=%lld N=%lld K=%lld (ldx %lld) not served", (long long)M, (long long)N, (long long)K,
              (long long)ldx);
    return MINITP_ERR_UNSUPPORTED;
  }
  if (swiglu) return launch_tile<TILE_SWIGLU>(st, x, ldx, w, nullptr, y, ldy, M, N, K, tail);
  return launch_tile<TILE_STORE>(st, x, ldx, w, bias, y, ldy, M, N, K, tail);
}

}  // namespace minitp
