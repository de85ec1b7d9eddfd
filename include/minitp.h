/*
 * minitp: C ABI of the MI355X (gfx950) Qwen2 token-loop library.
 *
 * Every entry point returns an int status (MINITP_OK == 0, negative on
 * error), never throws or aborts across the ABI, only borrows caller-owned
 * device pointers for the stream-ordered lifetime of the call, and never
 * allocates device memory (scratch comes from a caller workspace sized by
 * the matching *_workspace_bytes query). `stream` is a hipStream_t passed as
 * void*. Tensors are row-major; `dtype` is MINITP_F32 or MINITP_BF16 and
 * applies to every floating-point tensor of a call except the RoPE tables,
 * which are always fp32 (minitp/rope.py:34-35 keeps them in fp32).
 *
 * Citations are file:line in the mini-tp reference; each names the
 * reference function the entry point stands in for at tp_size == 1.
 */
#ifndef MINITP_H
#define MINITP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MINITP_ABI_VERSION 5

enum {
  MINITP_OK = 0,
  MINITP_ERR_ARG = -1,         /* bad pointer, shape, alignment or dtype   */
  MINITP_ERR_HIP = -2,         /* a HIP runtime call failed                */
  MINITP_ERR_OVERFLOW = -3,    /* KV cache overflow (kv_cache.py:49-52)    */
  MINITP_ERR_RANGE = -4,       /* index out of range (rope.py:37-45)       */
  MINITP_ERR_UNSUPPORTED = -5, /* valid request this build does not serve  */
  MINITP_ERR_DIVISIBLE = -6    /* TP divisibility (config.py:56-68)        */
};

enum { MINITP_F32 = 0, MINITP_BF16 = 1 };

/* Linear epilogues (see minitp_linear). */
enum {
  MINITP_EPI_NONE = 0,   /* y = x W^T (+ bias)                                     */
  MINITP_EPI_RESID = 1,  /* y = aux + (x W^T), each rounded to dtype (layer.py:63-64) */
  MINITP_EPI_SWIGLU = 2  /* W is [2N, K] = [gate; up]; y = silu(gate) * up (mlp.py:38) */
};

const char* minitp_status_string(int status);
/* Detail message of the last error raised on the calling thread. */
const char* minitp_last_error(void);
int minitp_abi_version(void);

/* ---- synthetic initialisation (seeded, bit-identical to the CPU spec) ---- */
/* dst[i] = dtype(float32(std * z_i)), z from the polar-method normal stream. */
int minitp_fill_normal(void* stream, int dtype, void* dst, int64_t count, uint64_t seed,
                       uint64_t stream_id, double std_dev);
/* dst[i] = uniform integer in [0, vocab). */
int minitp_fill_uniform_ids(void* stream, int64_t* dst, int64_t count, uint64_t seed,
                            uint64_t stream_id, int64_t vocab);
/* dst[i] = value (KVCache.poison, kv_cache.py:60-63; zeros init, kv_cache.py:33). */
int minitp_fill(void* stream, int dtype, void* dst, int64_t count, float value);

/* ---- elementwise / normalisation ---------------------------------------- */
/* VocabParallelEmbedding.forward at tp=1: F.embedding (embedding.py:44-46).
 * out[n, :] = table[ids[n], :]; an id outside [0, vocab) yields a NaN row. */
int minitp_embedding(void* stream, int dtype, const void* table, const int64_t* ids, void* out,
                     int64_t n_tokens, int64_t hidden, int64_t vocab);
/* RMSNorm.forward "reference" math (layer.py:39-42), fp32 internally:
 * out = dtype((x * rsqrt(mean(x^2) + eps)) * w). x, out: [rows, hidden]. */
int minitp_rmsnorm(void* stream, int dtype, const void* x, const void* w, void* out, int64_t rows,
                   int64_t hidden, float eps);
/* Residual add in the model dtype (layer.py:63-64): out[i] = dtype(a[i] + b[i % b_period]).
 * b_period == n is elementwise; b_period == hidden broadcasts one row (the
 * post-reduce bias add of RowParallelLinear, linear.py:120-121). */
int minitp_add(void* stream, int dtype, const void* a, const void* b, void* out, int64_t n, int64_t b_period);
/* SwiGLU gate (mlp.py:38): out = dtype(dtype(silu(gate)) * up).
 * gate/up rows have stride ld_in, out rows stride ld_out; [rows, n]. */
int minitp_silu_mul(void* stream, int dtype, const void* gate, const void* up, int64_t ld_in,
                    void* out, int64_t ld_out, int64_t rows, int64_t n);

/* Tensor.to(torch.bfloat16) of fp32 values (the casts of layer.py:42,
 * mlp.py:38, rope.py:62 ...): out[i] = round-to-nearest-even bf16 of in[i],
 * NaN stays NaN. */
int minitp_cast_f32_bf16(void* stream, const float* in, void* out, int64_t n);

/* ---- linear layers ------------------------------------------------------ */
/* F.linear(x, W, bias) with fp32 accumulation (linear.py:57-58, 111-122;
 * fused.py:57-61, 102-104), result rounded to dtype, then the epilogue.
 * x: [M, K] (row stride ldx), W: [N, K] (or [2N, K] for SWIGLU), bias: [N]
 * or NULL, y: [M, N] (row stride ldy), aux: [M, N] (stride ldy) for RESID
 * (may alias y). Small M streams W once as a GEMV (M <= 4; bf16 up to 32
 * rows on MFMA); larger M runs an MFMA GEMM. K must be a multiple of 8;
 * pointers 16-byte aligned. SWIGLU is served for the GEMV shapes and for
 * bf16 products of at least 96 output tiles of 256 rows x 128 columns (no
 * bias). */
int minitp_linear(void* stream, int dtype, const void* x, int64_t ldx, const void* w,
                  const void* bias, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                  int epilogue, const void* aux);
/* RMSNorm (layer.py:39-42) feeding a linear (the decoder layer's
 * input_layernorm -> qkv_proj and post_attention_layernorm -> gate_up_proj,
 * layer.py:60-67) in one pass over W: every block normalises the x rows it
 * needs (fp32, rounded to dtype) and streams its share of W. Arguments as
 * minitp_linear plus norm_w [K] and eps. Serves the decode shapes only
 * (M <= 4 rows, M == 1 up to K = 20480; bf16 5..32 rows up to K = 1024);
 * others return
 * MINITP_ERR_UNSUPPORTED (use minitp_rmsnorm, then minitp_linear). The norm
 * sums x^2 in a different order than minitp_rmsnorm, so the two agree to
 * rounding, not bitwise. */
int minitp_rmsnorm_linear(void* stream, int dtype, const void* x, int64_t ldx, const void* norm_w,
                          float eps, const void* w, const void* bias, void* y, int64_t ldy, int64_t M,
                          int64_t N, int64_t K, int epilogue, const void* aux);

/* The decoder layer's residual add, post_attention_layernorm and gate_up_proj
 * with SwiGLU for one row (layer.py:63-67, mlp.py:34-38), where the o_proj
 * product arrives as nparts fp32 partial rows over disjoint parts of its K
 * (the per-head partials of the batch-1 decode attention, which folds o_proj
 * in): x_out = dtype(x + dtype(parts[0] + parts[1] + ... in row order)), then
 * y = silu(gate) * up of RMSNorm(x_out) W^T as minitp_rmsnorm_linear.
 * x, x_out: [K]; parts: [nparts, K] fp32; W: [2N, K]; y: [N]. epilogue must be
 * MINITP_EPI_SWIGLU; K <= 1024, 1 <= nparts <= 16, else
 * MINITP_ERR_UNSUPPORTED. */
int minitp_add_rmsnorm_linear_parts(void* stream, int dtype, const void* x, const float* parts, int32_t nparts,
                                    void* x_out, const void* norm_w, float eps, const void* w, void* y,
                                    int64_t N, int64_t K, int epilogue);

/* ---- rotary embedding and KV cache -------------------------------------- */
/* RotaryEmbedding.apply (rope.py:47-64): q [B, Hq, T, D] and k [B, Hkv, T, D]
 * (contiguous) rotated by rows positions[t] of the fp32 tables [max_pos, D];
 * rotate_half pairs (i, i + D/2). Results go to q_out / k_out. Positions are
 * not range-checked here (the caller checks; rope.py:37-45). */
int minitp_rope(void* stream, int dtype, const void* q, const void* k, void* q_out, void* k_out,
                const float* cos_tab, const float* sin_tab, const int64_t* positions, int64_t B,
                int64_t Hq, int64_t Hkv, int64_t T, int64_t D);
/* KVCache.update write half (kv_cache.py:53-54): copy k_new / v_new
 * [B, H, T, D] (contiguous) into cache[b, h, cache_len + t, :] of the layer
 * buffers [B, H, S, D]. Returns MINITP_ERR_OVERFLOW if cache_len + T > S. */
int minitp_kv_write(void* stream, int dtype, const void* k_new, const void* v_new, void* k_cache,
                    void* v_cache, int64_t B, int64_t H, int64_t T, int64_t D, int64_t S,
                    int64_t cache_len);
/* Fused QKV split + RoPE + KV write (fused.py:60, attention.py:59-73):
 * qkv [B*T, (Hq+2Hkv)*D] (row stride ld_qkv, bias already added) ->
 * q_out [B, T, Hq, D] rotated, k rotated and v copied into the layer caches
 * [B, Hkv, S, D] at cache_len + t. Out-of-table positions give NaN rows. */
int minitp_rope_kv_write(void* stream, int dtype, const void* qkv, int64_t ld_qkv, void* q_out,
                         void* k_cache, void* v_cache, const float* cos_tab, const float* sin_tab,
                         const int64_t* positions, int64_t max_pos, int64_t B, int64_t T,
                         int64_t Hq, int64_t Hkv, int64_t D, int64_t S, int64_t cache_len);

/* ---- attention ---------------------------------------------------------- */
/* GQA scaled-dot-product attention over the cache (attention.py:77-105):
 * q [B, T, Hq, D]; caches [B, Hkv, S, D] hold cache_len + T valid rows;
 * query t of head h attends keys 0..cache_len + t of KV head h / (Hq/Hkv)
 * (T == 1: all keys; cache_len == 0: is_causal; else tril(diagonal=cache_len)).
 * out [B, T, Hq * D]. Scale 1/sqrt(D). Workspace from the query below. */
int64_t minitp_attention_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                         int64_t S);
int minitp_attention(void* stream, int dtype, const void* q, const void* k_cache,
                     const void* v_cache, void* out, int64_t B, int64_t T, int64_t Hq,
                     int64_t Hkv, int64_t D, int64_t S, int64_t cache_len, void* workspace,
                     int64_t workspace_bytes);

/* ---- greedy selection --------------------------------------------------- */
/* distributed_argmax tp=1 fast path (embedding.py:146-147; generation.py:59):
 * out[b * out_stride] = argmax over logits[b * ld + 0 .. V), torch.argmax
 * order (first maximum; NaN wins). Workspace from the query below. */
int64_t minitp_argmax_workspace_bytes(int64_t B, int64_t V);
int minitp_argmax(void* stream, int dtype, const void* logits, int64_t ld, int64_t B, int64_t V,
                  int64_t* out, int64_t out_stride, void* workspace, int64_t workspace_bytes);
/* minitp_argmax without a workspace: no counterpart in the reference. For
 * callers that cannot allocate device memory (code under hipGraph capture,
 * serving loops, harnesses that forbid hipMalloc). The slice partials live in
 * a static device array of minitp_argmax_static_max_bytes() bytes (1 MiB) per
 * device, held until the process ends; the call allocates nothing. Requests
 * needing more (B * ceil(V / 4096) * 12 bytes) return MINITP_ERR_ARG. Every
 * call on one device shares that device's array: calls that overlap on one
 * device (other streams, other threads) race and must be serialised by the
 * caller. Same arguments and results as minitp_argmax. */
int64_t minitp_argmax_static_max_bytes(void);
int minitp_argmax_static(void* stream, int dtype, const void* logits, int64_t ld, int64_t B, int64_t V,
                         int64_t* out, int64_t out_stride);

/* ---- whole-model programs ------------------------------------------------ */
/* TPQwen2ForCausalLM (layer.py:68-124) at tp_size == 1, run as one native
 * launch sequence; the decode step can be replayed as one hipGraph. */
typedef struct minitp_qwen2_config {
  int32_t dtype;
  int32_t num_layers;
  int32_t hidden;
  int32_t heads;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t intermediate;
  int32_t vocab;
  int32_t max_pos; /* rows of the RoPE tables */
  float eps;
} minitp_qwen2_config;

/* Per-layer pointer order in `layers` (7 per layer). */
enum {
  MINITP_W_LN1 = 0,
  MINITP_W_LN2 = 1,
  MINITP_W_QKV = 2,
  MINITP_W_QKV_BIAS = 3,
  MINITP_W_O = 4,
  MINITP_W_GATE_UP = 5,
  MINITP_W_DOWN = 6,
  MINITP_W_PER_LAYER = 7
};

typedef struct minitp_qwen2_weights {
  const void* embed;      /* [V, H] */
  const void* lm_head;    /* [V, H]; equals embed when tied (layer.py:88-89) */
  const void* final_norm; /* [H] */
  const float* rope_cos;  /* [max_pos, D] fp32 */
  const float* rope_sin;
  const void* const* layers; /* [num_layers * MINITP_W_PER_LAYER] */
} minitp_qwen2_weights;

/* One forward over ids [B, T]. logits: [B, T, V] when logits_all, else the
 * last position only [B, V]. next_tok (optional): argmax of the last
 * position per row, written to next_tok[b * next_tok_ld]. The KV caches are
 * [L, B, Hkv, S, D]; rows cache_len .. cache_len + T - 1 are written.
 *
 * End-of-sequence early stop kept on the device (generate_greedy's
 * finished mask, generation.py:150-168), on when eos_state is not NULL
 * (next_tok required): after the token selection, a row that had finished
 * gets eos_token, and a row finishes when its token is eos_token. eos_state
 * is device memory of batch + 2 int64 words, zero before the first forward
 * of a generation: the finished flags, then a halted word, then the stop
 * column. When every row has finished, the forward sets halted and the stop
 * column to cursor + 1 (cursor = the column next_tok points into: the
 * reference's cursor after the append that ends its loop), and stores the
 * stop column to *eos_host too when that is not NULL (a device address of
 * pinned host memory, minitp_host_device_pointer). Forwards run after the
 * halt write no KV rows, change no token and no flag: a host that checks the
 * stop column a few steps late loses nothing but time. */
typedef struct minitp_qwen2_step {
  const int64_t* ids;
  int64_t ids_ld;
  const int64_t* positions; /* [T] absolute positions */
  int64_t batch;
  int64_t tokens;
  int64_t cache_len;
  void* k_cache;
  void* v_cache;
  int64_t max_seq;
  void* logits;
  int32_t logits_all;
  int64_t* next_tok;
  int64_t next_tok_ld;
  void* workspace;
  int64_t workspace_bytes;
  int64_t* eos_state;
  int64_t eos_token;
  int64_t cursor;
  int64_t* eos_host;
} minitp_qwen2_step;

/* Device address of pinned host memory (hipHostMalloc / torch pin_memory),
 * for eos_host. No counterpart in the reference (its host reads a device
 * flag with a blocking copy each step). */
int minitp_host_device_pointer(void* host, void** device);

int minitp_qwen2_create(const minitp_qwen2_config* cfg, const minitp_qwen2_weights* w,
                        void** handle);
int minitp_qwen2_destroy(void* handle);
/* Workspace for forwards of up to max_tokens = B*T rows, batch B, cache S.
 * A workspace must be zero-filled once before its first use (its first
 * bytes hold the step state: the error word and the arrival words of the
 * split products, which every launch leaves at zero) and then only be used
 * with this handle. */
int64_t minitp_qwen2_workspace_bytes(void* handle, int64_t max_tokens, int64_t batch,
                                     int64_t max_seq);
/* GenerationState.prefill / TPQwen2ForCausalLM.forward (generation.py:112-117,
 * layer.py:91-124): direct launches. */
int minitp_qwen2_forward(void* handle, void* stream, const minitp_qwen2_step* step);
/* GenerationState.decode_step (generation.py:129-130): one T == 1 forward,
 * replayed from a hipGraph captured on first use for (batch, max_seq,
 * workspace), with per-step scalars and pointers patched into the graph's
 * first node. */
int minitp_qwen2_decode(void* handle, void* stream, const minitp_qwen2_step* step);
/* Out-of-range RoPE positions (rope.py:37-45, where the reference's gather
 * raises): a forward whose position lies outside the table computes with NaN
 * rotary rows and sets a sticky error word in its workspace, because a
 * graph-replayed step cannot return a status for a value that lives on the
 * device. This waits for `stream`, returns MINITP_ERR_RANGE if any forward
 * on `workspace` since the last check set the word, and clears it. */
int minitp_qwen2_decode_check(void* handle, void* stream, void* workspace);

#ifdef __cplusplus
}
#endif

#endif /* MINITP_H */
