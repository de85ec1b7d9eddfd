// Host-side launch interface of the minitp kernels (internal to the library).
#pragma once

#include "common.h"

namespace minitp {

// Per-forward scalars and pointers the decode sequence reads from device
// memory, so a captured hipGraph stays valid from step to step: only the
// first node's arguments change, and it writes this struct.
constexpr int MAX_HEAD_DIM = 128;

// Per-forward scalars and pointers (passed by value to the first kernel).
struct StepArgs {
  const int64_t* ids;  // [B, T] token ids, row stride ids_ld
  int64_t ids_ld;
  const int64_t* positions;  // [T]
  int64_t cache_len;         // KV rows already filled
  void* k_cache;             // [L, B, Hkv, S, D]
  void* v_cache;
  void* logits;  // [B, V] (or [B, T, V]) logits output
  int64_t* next_tok;
  int64_t next_tok_ld;
  // end-of-sequence early stop (NULL eos_state: off); words of eos_state:
  // [0, B) finished flags, B halted, B + 1 stop column
  int64_t* eos_state;
  int64_t eos_token;
  int64_t cursor;     // column of the output ids that next_tok points into
  int64_t* eos_host;  // device address of a pinned host word, or NULL
};

// What the forward's later kernels read from device memory, so a captured
// hipGraph stays valid from step to step: only the first node's arguments
// change, and that node writes this struct.
// Tuples (4 output rows each) and K segments of one split-K GEMV launch.
constexpr int SPLIT_MAX_TUPLES = 2048;
constexpr int SPLIT_MAX_SEG = 8;

struct StepState {
  StepArgs args;
  int32_t error;   // 1: a position was outside the RoPE table
  int32_t halted;  // early stop reached before this forward: no KV writes
  // T == 1: the RoPE table rows of positions[0], copied by the first kernel of
  // the forward so the QKV epilogue reads them at a fixed address (NaN when
  // the position is outside the table).
  float rope_cos[MAX_HEAD_DIM];
  float rope_sin[MAX_HEAD_DIM];
  // arrival words of the split-K GEMV, zeroed by the first kernel of every
  // forward (each launch also leaves them at 0)
  uint32_t split_count[SPLIT_MAX_TUPLES];
};

// Layer-independent shape of the attention / KV layout.
struct AttnShape {
  int B, T, Hq, Hkv, D;
  int64_t S;  // cache capacity per (b, kv head)
};

// PRO_PART_NORM (one input row): the input is x + the sum of `nparts` fp32
// partial rows of a product split over K (the per-head o_proj partials of the
// fused attention), rounded like the residual add of layer.py:63 before the
// RMSNorm; block 0 also stores that row to x_out.
enum GemvPro { PRO_NONE = 0, PRO_NORM = 1, PRO_PART_NORM = 2 };
enum GemvEpi { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKV_ROPE = 3, EPI_ARGMAX = 4 };

struct GemvArgs {
  const void* x;  // [M, K] input rows (pre-norm residual when PRO_NORM)
  int64_t ldx;
  const void* norm_w;  // [K] RMSNorm weight (PRO_NORM)
  float eps;
  const void* w;     // weight rows, each K long
  const void* bias;  // [N] or null (EPI_STORE, EPI_QKV_ROPE)
  void* y;           // output [M, N] (row stride ldy)
  int64_t ldy;
  const void* aux;  // residual [M, N] (EPI_RESID; may alias y)
  int64_t M, N, K;  // N: logical outputs (EPI_SWIGLU: weight has 2N rows)
  // EPI_QKV_ROPE: q -> y as [B, T, Hq, D]; k, v -> caches of layer `layer`
  const StepState* st;
  const float* cos_tab;
  const float* sin_tab;
  int64_t max_pos;
  int layer;
  AttnShape a;
  // EPI_ARGMAX: logits -> st->logits (ld N), token -> st->next_tok (through
  // argmax_merge_kernel, launched right after the GEMV)
  float* part_val;  // [M, gridDim.x] block partials
  int64_t* part_idx;
  // Split-K form (rows longer than the register path holds): fp32 segment
  // partials [tuples, segments, M, 4] and one arrival word per tuple, 0
  // between launches. Both null: the split form is not used.
  float* split_part;
  uint32_t* split_count;
  int64_t split_part_bytes;
  // PRO_PART_NORM: partial rows [nparts][K] fp32 and where block 0 writes x + their sum
  const float* part;
  int nparts;
  void* x_out;
  int max_grid;  // register form: cap on the grid (0: the default)
};

// gemv.hip
// The partial-sum prologue's limits: at most PART_MAX_PARTS partial rows of
// K <= PART_MAX_K elements (one row).
constexpr int PART_MAX_PARTS = 16;
constexpr int64_t PART_MAX_K = 1024;
bool gemv_part_supported(int dtype, int64_t K, int nparts);
// RMSNorm(x + sum of partials) -> gate/up -> SwiGLU for one row (PRO_PART_NORM, EPI_SWIGLU)
int launch_gemv_part_swiglu(hipStream_t st, int dtype, const GemvArgs& a);
int64_t gemv_argmax_partials(int64_t N);
int launch_gemv(hipStream_t st, int dtype, int pro, int epi, const GemvArgs& a);
bool gemv_supported(int dtype, int64_t M, int64_t K);
// bf16 rows MF_MIN_ROWS..32 run the MFMA forms (16-row operand tiles, rows
// past M read as zeros); fewer rows and fp32 the register forms. At 3 and 4
// rows the register forms' per-lane row budget leaves long rows (the 0.5B
// down projection, K = 4,864) to the prompt GEMM: 0.5B decode at batch 4
// took 1.44 ms a step that way, batch 5 on the MFMA forms 0.92.
constexpr int MF_MIN_ROWS = 3;
inline bool gemv_mfma_rows(int dtype, int64_t M) { return dtype == MINITP_BF16 && M >= MF_MIN_ROWS && M <= 32; }
// Bytes of GemvArgs::split_part for products of M input rows (the register
// form's SPLIT_MAX_TUPLES x SPLIT_MAX_SEG x 4 x 4 floats; 16 MiB for the
// MFMA form's 16 x 32 tiles).
int64_t gemv_split_part_bytes(int64_t M);
// ... and with the RMSNorm prologue (PRO_NORM)
bool gemv_norm_supported(int dtype, int64_t M, int64_t K);

// gemm.hip: y[M, N] = epilogue(x[M, K] W[N, K]^T (+ bias)), MFMA tiles.
// When `state` is non-null the output base is state->logits (graph replays).
// With a workspace (ws, ws_bytes), small-M products split K over more
// blocks and reduce the fp32 partials in a second kernel.
// GEMM workspace of a forward: the split-K partials of launch_gemm use the
// first GEMM_SPLIT_BYTES (launch_gemm_partials may take all of it); the
// tile GEMM's split of its last, partial round over K (TileTail) takes the
// next TILE_TAIL_BYTES.
constexpr int64_t GEMM_SPLIT_BYTES = 8LL << 20;
constexpr int64_t TILE_TAIL_BYTES = 64LL << 20;
constexpr int64_t GEMM_WS_BYTES = GEMM_SPLIT_BYTES + TILE_TAIL_BYTES;
// fp32 partials and arrival words (zero between launches) for the tile
// GEMM's split last round; null members: no split
struct TileTail {
  float* part;
  uint32_t* count;
};
int launch_gemm(hipStream_t st, int dtype, const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                int64_t ldy, int64_t M, int64_t N, int64_t K, int epi, const void* aux,
                const StepState* state = nullptr, void* ws = nullptr, int64_t ws_bytes = 0,
                TileTail tail = TileTail{nullptr, nullptr});
// The first half of a bf16 product that launch_gemm would split over K: the
// split GEMM alone, its fp32 partials [S][M][N] in ws (described in *out),
// for a consumer kernel to add up in split order with its own epilogue
// (the *_partials launchers). MINITP_ERR_UNSUPPORTED when the product is
// not split (tile kernel, one split, fp32): the caller runs launch_gemm.
int launch_gemm_partials(hipStream_t st, int dtype, const void* x, int64_t ldx, const void* w, int64_t M, int64_t N,
                         int64_t K, void* ws, int64_t ws_bytes, Partials* out, int64_t target_blocks = 0);
// bf16 y[M, N] = swiglu(x W_gate^T, x W_up^T) for W = [gate; up] ([2N, K]) on
// the small tiles, unsplit (M < 512), gate and up rounded to bf16 first as
// launch_gemm + launch_silu_mul would store and read them
int launch_gemm_swiglu(hipStream_t st, int dtype, const void* x, int64_t ldx, const void* w, void* y, int64_t ldy,
                       int64_t M, int64_t N, int64_t K);

// gemm_tile.hip: 256 x 256 MFMA tiles (32x32x16 bf16) for prompt-sized
// bf16 products; swiglu: W is [2N, K] = [gate; up] and y = silu(gate) * up
// [M, N]. MINITP_ERR_UNSUPPORTED for shapes it does not serve (too few
// tiles, operands past 4 GiB, unaligned rows).
bool gemm_tile_supported(int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy, bool swiglu);
int launch_gemm_tile(hipStream_t st, const void* x, int64_t ldx, const void* w, const void* bias, void* y, int64_t ldy,
                     int64_t M, int64_t N, int64_t K, bool swiglu, TileTail tail = TileTail{nullptr, nullptr});
// The same tiles for products with too few of them (M a multiple of 256,
// fewer tiles than half the CUs) and a long K: every tile split over K into
// parts that its last block adds (needs the forward's tail buffers)
bool gemm_tile_split_supported(int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy, bool swiglu);
int launch_gemm_tile_split(hipStream_t st, const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                           int64_t ldy, int64_t M, int64_t N, int64_t K, bool swiglu, TileTail tail);

// elementwise.hip
int launch_fill_normal(hipStream_t st, int dtype, void* dst, int64_t count, uint64_t seed, uint64_t sid,
                       double std_dev);
int launch_fill_ids(hipStream_t st, int64_t* dst, int64_t count, uint64_t seed, uint64_t sid, int64_t vocab);
int launch_fill(hipStream_t st, int dtype, void* dst, int64_t count, float value);
int launch_embedding(hipStream_t st, int dtype, const void* table, const int64_t* ids, int64_t ids_ld, int64_t B,
                     int64_t T, void* out, int64_t hidden, int64_t vocab);
int launch_rmsnorm(hipStream_t st, int dtype, const void* x, const void* w, void* out, int64_t rows, int64_t hidden,
                   float eps);
int launch_add(hipStream_t st, int dtype, const void* a, const void* b, void* out, int64_t n, int64_t b_period);
int launch_silu_mul(hipStream_t st, int dtype, const void* gate, const void* up, int64_t ld_in, void* out,
                    int64_t ld_out, int64_t rows, int64_t n);
int launch_cast_f32_bf16(hipStream_t st, const float* in, void* out, int64_t n);
int launch_add_rmsnorm(hipStream_t st, int dtype, void* x, const void* delta, const void* w, void* out, int64_t rows,
                       int64_t hidden, float eps);
// bf16 launch_add_rmsnorm / launch_silu_mul whose delta / [gate, up] input is
// a split product's partials (the sums rounded to bf16 as launch_gemm
// stores them, so the results are the same bits)
int launch_add_rmsnorm_partials(hipStream_t st, void* x, const Partials& delta, const void* w, void* out,
                                int64_t hidden, float eps);
int launch_silu_mul_partials(hipStream_t st, const Partials& gu, void* out, int64_t ld_out, int64_t n);

// rope.hip
int launch_rope(hipStream_t st, int dtype, const void* q, const void* k, void* q_out, void* k_out, const float* cos_tab,
                const float* sin_tab, const int64_t* positions, int64_t B, int64_t Hq, int64_t Hkv, int64_t T,
                int64_t D);
int launch_kv_write(hipStream_t st, int dtype, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                    int64_t B, int64_t H, int64_t T, int64_t D, int64_t S, int64_t cache_len);
int launch_rope_kv_write(hipStream_t st, int dtype, const void* qkv, int64_t ld_qkv, void* q_out, void* k_cache,
                         void* v_cache, const float* cos_tab, const float* sin_tab, const int64_t* positions,
                         int64_t max_pos, int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t S,
                         int64_t cache_len, int32_t* error_flag, const StepState* state = nullptr,
                         int layer = 0);
// bf16 launch_rope_kv_write of a QKV projection given as its split partials
// plus the bias (positions, cache length and caches from the step state)
int launch_rope_kv_write_partials(hipStream_t st, const Partials& qkv, const void* bias, void* q_out,
                                  const float* cos_tab, const float* sin_tab, int64_t max_pos, int64_t B, int64_t T,
                                  int64_t Hq, int64_t Hkv, int64_t D, int64_t S, const StepState* state, int layer);

// attention.hip. Decode (T == 1) may read cache_len and the cache bases
// from a StepState (graph replay); prefill takes them by value.
int64_t attention_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t S);
int launch_decode_attention(hipStream_t st, int dtype, const void* q, const void* k_cache, const void* v_cache,
                            void* out, const AttnShape& a, int64_t cache_len, const StepState* state, int layer,
                            void* workspace, int64_t workspace_bytes);
// Decode attention of one batch row with the o_proj product folded in
// (attention.py:77-105 then o_proj, attention.py:42-44 / linear.py:117):
// block (query head h, row slice r) runs head h's attention, rounds its
// output to the dtype and multiplies it by W_o[rows of slice r, h * D ..
// h * D + D), storing the fp32 partial part[h][rows]. Summed over h (in
// head order) by the next kernel's prologue. Cache and cache_len from the
// step state. One batch row; served when attn_oproj_supported says so.
struct OprojArgs {
  const void* w;   // W_o [H, Hq * D]
  int64_t H;       // output rows
  int rows;        // rows per slice (gridDim.y = ceil(H / rows))
  float* part;     // [Hq][H]
};
// W_o row slices a model asks for: more slices re-run each head's attention
// more often but give each block fewer rows (0.5B: 4 slices 0.524 ms a
// token, 8 0.518, 16 0.517; with the later kernels 16 0.502, 18 0.503, 32
// 0.533).
constexpr int OPROJ_SLICES = 16;
bool attn_oproj_supported(int dtype, const AttnShape& a, int64_t H, int slices);
int attn_oproj_rows(int dtype, const AttnShape& a, int64_t H, int slices);
int launch_decode_attention_oproj(hipStream_t st, int dtype, const void* q, const AttnShape& a,
                                  const StepState* state, int layer, const OprojArgs& o);
// Inside a forward (state != null) the caches of layer `layer` and cache_len
// come from the step state (k_cache, v_cache and cache_len unused).
int launch_prefill_attention(hipStream_t st, int dtype, const void* q, const void* k_cache, const void* v_cache,
                             void* out, const AttnShape& a, int64_t cache_len, const StepState* state = nullptr,
                             int layer = 0);

// argmax.hip
int64_t argmax_workspace_bytes(int64_t B, int64_t V);
// The argmax with its partials in the library's static device scratch.
int64_t argmax_static_scratch_bytes();
int launch_argmax_static(hipStream_t st, int dtype, const void* logits, int64_t ld, int64_t B, int64_t V, int64_t* out,
                         int64_t out_stride);
// Winner of each of `rows` rows of nb (value, index) partials -> out (or
// state->next_tok when state is non-null; nothing when that is null).
// End-of-sequence bookkeeping after a forward's token selection (one block).
int launch_eos_update(hipStream_t st, const StepState* state, int64_t B);
int launch_argmax_merge(hipStream_t st, const float* pv, const int64_t* pi, int64_t nb, int64_t rows, int64_t* out,
                        int64_t out_stride, const StepState* state);
// With `state`: logits = state->logits + row_offset, out = state->next_tok
// (stride state->next_tok_ld); row b of the logits starts at b * ld.
int launch_argmax(hipStream_t st, int dtype, const void* logits, int64_t ld, int64_t B, int64_t V, int64_t* out,
                  int64_t out_stride, void* workspace, int64_t workspace_bytes, const StepState* state = nullptr,
                  int64_t row_offset = 0);

// Raise the dynamic-LDS limit of a kernel once (needed above 64 KiB).
int ensure_lds_limit(const void* kernel, int bytes);

}  // namespace minitp
