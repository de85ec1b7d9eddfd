// Whole-model Qwen2 program at tp_size == 1: TPQwen2ForCausalLM.forward
// (layer.py:91-124) as one native launch sequence, and the decode step as a
// replayable hipGraph.
//
// Per-forward values (ids, positions, cache cursor, cache / logits / token
// pointers) travel in a StepState that the first kernel writes into the
// workspace; every later kernel reads it from there. A captured decode graph
// therefore never needs re-capture: each replay patches only the first
// node's by-value argument.
//
// Rows M = B * T <= 4 take the fused GEMV path, 5 kernels per layer:
//   [RMSNorm -> QKV + bias -> RoPE -> q, KV write] [attention]
//   [o_proj + residual] [RMSNorm -> gate/up -> SwiGLU] [down + residual]
// and the final RMSNorm -> LM head -> argmax is one more kernel. Larger M
// runs MFMA GEMMs with separate norm / RoPE / SwiGLU kernels.
#include <cmath>
#include <cstddef>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"
#include "kernels.h"

#ifndef MINITP_DOWN_TILE_SPLIT
#define MINITP_DOWN_TILE_SPLIT 1
#endif
#ifndef MINITP_GEMM_SWIGLU_EPI
#define MINITP_GEMM_SWIGLU_EPI 1
#endif

namespace minitp {

namespace {

// First kernel of every forward: publishes the per-forward values (StepState)
// for the rest of the sequence, copies the RoPE rows of a single-token
// forward's position next to them, and gathers the embedding rows
// (embedding.py:44-46). The error word is sticky: a position outside the
// RoPE table sets it, and only minitp_qwen2_decode_check clears it.
template <typename T>
__global__ void step_embed_kernel(StepState* dst, StepArgs val, const T* __restrict__ table, T* __restrict__ out,
                                  int64_t hidden, int64_t vocab, int64_t T_, const float* cos_tab,
                                  const float* sin_tab, int64_t max_pos, int head_dim) {
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i < SPLIT_MAX_TUPLES; i += blockDim.x) dst->split_count[i] = 0u;
    if (threadIdx.x == 0) {
      dst->args = val;
      dst->halted = val.eos_state != nullptr && val.eos_state[gridDim.x / T_] != 0;
    }
    if (T_ == 1) {
      const int64_t pos = val.positions[0];
      const bool ok = pos >= 0 && pos < max_pos;
      for (int i = threadIdx.x; i < head_dim; i += blockDim.x) {
        dst->rope_cos[i] = ok ? cos_tab[pos * head_dim + i] : __builtin_nanf("");
        dst->rope_sin[i] = ok ? sin_tab[pos * head_dim + i] : __builtin_nanf("");
      }
      if (!ok && threadIdx.x == 0) dst->error = 1;
    }
  }
  const int64_t n = blockIdx.x, b = n / T_, t = n % T_;
  const int64_t id = val.ids[b * val.ids_ld + t];
  T* o = out + n * hidden;
  if (id < 0 || id >= vocab) {
    for (int64_t i = threadIdx.x; i < hidden; i += blockDim.x) store_f32<T>(o, i, __builtin_nanf(""));
    return;
  }
  const uint4* src = reinterpret_cast<const uint4*>(table + id * hidden);
  uint4* d4 = reinterpret_cast<uint4*>(o);
  const int64_t nv = hidden * (int64_t)sizeof(T) / 16;
  for (int64_t i = threadIdx.x; i < nv; i += blockDim.x) d4[i] = src[i];
}

constexpr int EMBED_THREADS = 128;

StepArgs step_args(const minitp_qwen2_step& s) {
  StepArgs val{};
  val.ids = s.ids;
  val.ids_ld = s.ids_ld;
  val.positions = s.positions;
  val.cache_len = s.cache_len;
  val.k_cache = s.k_cache;
  val.v_cache = s.v_cache;
  val.logits = s.logits;
  val.next_tok = s.next_tok;
  val.next_tok_ld = s.next_tok_ld;
  val.eos_state = s.eos_state;
  val.eos_token = s.eos_token;
  val.cursor = s.cursor;
  val.eos_host = s.eos_host;
  return val;
}

struct Ws {
  StepState* st;
  void *x, *h, *qkv, *q, *attn, *gu, *act;
  void* attn_ws;
  int64_t attn_ws_bytes;
  float* part_val;
  int64_t* part_idx;
  void* amax_ws;
  int64_t amax_ws_bytes;
  void* gemm_ws;  // split-K partials of the prefill / batched GEMMs
  float* split_part;  // segment partials of the split-K GEMVs
  int64_t split_part_bytes;
  uint32_t* split_count;  // their arrival words (in the StepState)
  float* opart;  // [Hq][H] fp32 o_proj partials of the fused attention (one row)
  int64_t bytes;
};

// What a prompt forward's launch sequence depends on (its graph key).
struct GraphKey {
  int64_t batch, tokens, max_seq;
  void* workspace;
  bool eos, pick, all;
  bool operator==(const GraphKey& o) const {
    return batch == o.batch && tokens == o.tokens && max_seq == o.max_seq && workspace == o.workspace &&
           eos == o.eos && pick == o.pick && all == o.all;
  }
};

struct GraphEntry {
  GraphKey key;  // eos: the end-of-sequence update after the token selection;
                 // pick: the token selection (next_tok set; batch > 4 has no pick
                 // node otherwise); all: every position's logits, not the last's
  hipGraph_t graph;
  hipGraphExec_t exec;
  hipGraphNode_t first;
  uint64_t last_use;         // call clock of the last replay (least recently used goes first)
  hipStream_t last_stream;   // stream of the last launch (waited on before a destroy)
};

// Calls seen per shape, recorded or not (the graph cache's admission test).
struct ShapeCalls {
  GraphKey key;
  uint64_t calls, last;
};

inline int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

}  // namespace

struct Qwen2Program {
  minitp_qwen2_config c;
  const void* embed;
  const void* lm_head;
  const void* final_norm;
  const float* cos_tab;
  const float* sin_tab;
  std::vector<const void*> lw;
  std::mutex mu;
  std::vector<GraphEntry> graphs;
  std::vector<ShapeCalls> shape_calls;  // calls per shape (at most 64 shapes tracked)
  uint64_t clock = 0;                  // forward calls through run_graphed
  hipStream_t capture_stream = nullptr;
  // bf16 prompt forwards (last-position logits) through a graph per shape;
  // direct launches when MINITP_PREFILL_GRAPH=0 is in the environment at
  // creation
  bool prefill_graphs = true;
  // batch-1 decode folds o_proj into the attention kernel (partials summed by
  // the gate/up prologue); MINITP_FUSE_OPROJ=0 at creation keeps the
  // separate o_proj GEMV
  bool fuse_oproj = true;

  int es() const { return c.dtype == MINITP_F32 ? 4 : 2; }
  int qkv_rows() const { return (c.heads + 2 * c.kv_heads) * c.head_dim; }
  int q_rows() const { return c.heads * c.head_dim; }
  const void* L(int layer, int which) const { return lw[(size_t)layer * MINITP_W_PER_LAYER + which]; }

  Ws layout(void* base, int64_t M, int64_t B, int64_t S) const {
    Ws w{};
    char* p = (char*)base;
    int64_t off = 0;
    auto take = [&](int64_t bytes) {
      char* r = p ? p + off : nullptr;
      off += align256(bytes);
      return (void*)r;
    };
    w.st = (StepState*)take(sizeof(StepState));
    w.x = take(M * c.hidden * es());
    w.h = take(M * c.hidden * es());
    w.qkv = take(M * qkv_rows() * es());
    w.q = take(M * q_rows() * es());
    w.attn = take(M * q_rows() * es());
    w.gu = take(M * 2LL * c.intermediate * es());
    w.act = take(M * (int64_t)c.intermediate * es());
    w.attn_ws_bytes = attention_workspace_bytes(B, 1, c.heads, c.kv_heads, c.head_dim, S);
    w.attn_ws = take(w.attn_ws_bytes);
    const int64_t np = gemv_argmax_partials(c.vocab);
    w.part_val = (float*)take(std::min<int64_t>(B, 4) * np * 4);
    w.part_idx = (int64_t*)take(std::min<int64_t>(B, 4) * np * 8);
    w.amax_ws_bytes = argmax_workspace_bytes(B, c.vocab);
    w.amax_ws = take(w.amax_ws_bytes);
    w.gemm_ws = take(GEMM_WS_BYTES);
    w.split_part_bytes = gemv_split_part_bytes(M);
    w.split_part = (float*)take(w.split_part_bytes);
    w.split_count = w.st ? (uint32_t*)((char*)w.st + offsetof(StepState, split_count)) : nullptr;
    w.opart = (float*)take((int64_t)c.heads * c.hidden * 4);
    w.bytes = off;
    return w;
  }

  // bf16 prompts replay a graph per shape when every kernel of their forward
  // reads the per-call values from the step state: all of them with the last
  // position's logits; with every position's logits, those whose LM head runs
  // launch_gemm (logits pointer from the state), not the GEMV form (few rows)
  // or the tile kernel (M >= 256), which store to the pointer they are given.
  bool prompt_graphable(const minitp_qwen2_step& s) const {
    if (!prefill_graphs || s.tokens <= 1 || c.dtype != MINITP_BF16) return false;
    if (!s.logits_all) return true;
    const int64_t M = s.batch * s.tokens;
    return !fused(M) && !gemm_tile_supported(M, c.vocab, c.hidden, c.hidden, c.vocab, false);
  }

  bool fused(int64_t M) const {
    return gemv_norm_supported(c.dtype, M, c.hidden) && gemv_supported(c.dtype, M, c.intermediate) &&
           gemv_supported(c.dtype, M, q_rows());
  }

  // The launch sequence of one forward (also what a decode graph records).
  int run(hipStream_t st, const minitp_qwen2_step& s, const Ws& w) {
    const int rc = run_model(st, s, w);
    if (rc || s.eos_state == nullptr) return rc;
    return launch_eos_update(st, w.st, s.batch);
  }

  int run_model(hipStream_t st, const minitp_qwen2_step& s, const Ws& w) {
    const int64_t B = s.batch, T = s.tokens, M = B * T;
    const int64_t H = c.hidden, I = c.intermediate, V = c.vocab;
    const int D = c.head_dim;
    int rc;
    const StepArgs val = step_args(s);
    const int64_t max_pos = c.max_pos;
    if (c.dtype == MINITP_F32)
      hipLaunchKernelGGL(step_embed_kernel<float>, dim3((unsigned)M), dim3(EMBED_THREADS), 0, st, w.st, val,
                         (const float*)embed, (float*)w.x, H, (int64_t)V, T, cos_tab, sin_tab, max_pos, D);
    else
      hipLaunchKernelGGL(step_embed_kernel<bf16>, dim3((unsigned)M), dim3(EMBED_THREADS), 0, st, w.st, val,
                         (const bf16*)embed, (bf16*)w.x, H, (int64_t)V, T, cos_tab, sin_tab, max_pos, D);
    MINITP_LAUNCH_CHECK();

    const bool fz = fused(M);
    AttnShape as{(int)B, (int)T, c.heads, c.kv_heads, D, s.max_seq};
    // one-row decode: attention + o_proj in one kernel, its per-head partials
    // summed (with the residual) by the gate/up prologue
    const bool fo = fz && T == 1 && fuse_oproj && attn_oproj_supported(c.dtype, as, H, OPROJ_SLICES) &&
                    gemv_part_supported(c.dtype, H, c.heads);
    const int64_t layer_elems = B * c.kv_heads * s.max_seq * D;
    // bf16 prompts: plain GEMMs (the 256 x 256 MFMA tile kernel where the
    // shape fills the chip, else the split-K one), gate/up with SwiGLU in
    // the tile kernel's epilogue. The residual adds go with the next RMSNorm
    // (one fused kernel, the reference's rounding order), the projections
    // that feed them writing into the normed-input buffer h, free at that
    // point.
    const bool blas = c.dtype == MINITP_BF16 && !fz && T > 1;
    // the tile GEMM's split last round: partials after the split-K region,
    // arrival words in the step state (zeroed by the embedding kernel)
    const TileTail tail{(float*)((char*)w.gemm_ws + GEMM_SPLIT_BYTES), w.split_count};
    auto lin = [&](const void* xin, int64_t ldx, const void* wt, const void* b, void* y, int64_t ldy, int64_t n,
                   int64_t k) -> int {
      return launch_gemm(st, c.dtype, xin, ldx, wt, b, y, ldy, M, n, k, MINITP_EPI_NONE, nullptr, nullptr, w.gemm_ws,
                         GEMM_SPLIT_BYTES, tail);
    };
    if (blas && (rc = launch_rmsnorm(st, c.dtype, w.x, L(0, MINITP_W_LN1), w.h, M, H, c.eps))) return rc;
    // Prompt products that the split-K GEMM serves hand their partials to
    // the kernel after them (RoPE + KV write, residual add + RMSNorm,
    // SwiGLU), which adds them up in split order: no reduction launch, and
    // the same bits as reduce-then-consume. The partials may take the whole
    // GEMM workspace (nothing else in it is live between the two launches).
    const bool fuse_split = blas && D % 16 == 0 && H % 8 == 0 && I % 8 == 0 &&
                            aligned16(cos_tab) && aligned16(sin_tab);
    auto partials = [&](const void* xin, int64_t ldx, const void* wt, int64_t n, int64_t k, Partials* p) -> int {
      if (!fuse_split) return MINITP_ERR_UNSUPPORTED;
      return launch_gemm_partials(st, c.dtype, xin, ldx, wt, M, n, k, w.gemm_ws, GEMM_WS_BYTES, p);
    };
    auto split_bufs = [&](GemvArgs& g) {
      g.split_part = w.split_part;
      g.split_part_bytes = w.split_part_bytes;
      g.split_count = w.split_count;
    };
    for (int l = 0; l < c.num_layers; ++l) {
      if (blas) {
        // h holds input_layernorm(x) of this layer
        Partials pp{};
        rc = partials(w.h, H, L(l, MINITP_W_QKV), qkv_rows(), H, &pp);
        if (rc == MINITP_OK) {
          rc = launch_rope_kv_write_partials(st, pp, L(l, MINITP_W_QKV_BIAS), w.q, cos_tab, sin_tab, c.max_pos, B, T,
                                             c.heads, c.kv_heads, D, s.max_seq, w.st, l);
        } else if (rc == MINITP_ERR_UNSUPPORTED) {
          rc = lin(w.h, H, L(l, MINITP_W_QKV), L(l, MINITP_W_QKV_BIAS), w.qkv, qkv_rows(), qkv_rows(), H);
          if (!rc)
            rc = launch_rope_kv_write(st, c.dtype, w.qkv, qkv_rows(), w.q, nullptr, nullptr, cos_tab, sin_tab, nullptr,
                                      c.max_pos, B, T, c.heads, c.kv_heads, D, s.max_seq, 0, nullptr, w.st, l);
        }
        if (rc) return rc;
        const char* kc = (const char*)s.k_cache + l * layer_elems * es();
        const char* vc = (const char*)s.v_cache + l * layer_elems * es();
        if ((rc = launch_prefill_attention(st, c.dtype, w.q, kc, vc, w.attn, as, s.cache_len, w.st, l))) return rc;
        // x += o_proj(attn), h = post_attention_layernorm(x)
        rc = partials(w.attn, q_rows(), L(l, MINITP_W_O), H, q_rows(), &pp);
        if (rc == MINITP_OK) {
          rc = launch_add_rmsnorm_partials(st, w.x, pp, L(l, MINITP_W_LN2), w.h, H, c.eps);
        } else if (rc == MINITP_ERR_UNSUPPORTED) {
          rc = lin(w.attn, q_rows(), L(l, MINITP_W_O), nullptr, w.h, H, H, q_rows());
          if (!rc) rc = launch_add_rmsnorm(st, c.dtype, w.x, w.h, L(l, MINITP_W_LN2), w.h, M, H, c.eps);
        }
        if (rc) return rc;
        if (gemm_tile_supported(M, I, H, H, I, true)) {
          if ((rc = launch_gemm_tile(st, w.h, H, L(l, MINITP_W_GATE_UP), nullptr, w.act, I, M, I, H, true, tail)))
            return rc;
        } else {
          rc = partials(w.h, H, L(l, MINITP_W_GATE_UP), 2 * I, H, &pp);
          if (rc == MINITP_OK) {
            rc = launch_silu_mul_partials(st, pp, w.act, I, I);
          } else if (rc == MINITP_ERR_UNSUPPORTED && MINITP_GEMM_SWIGLU_EPI) {
            // unsplit: SwiGLU in the GEMM's epilogue
            rc = launch_gemm_swiglu(st, c.dtype, w.h, H, L(l, MINITP_W_GATE_UP), w.act, I, M, I, H);
          }
          if (rc == MINITP_ERR_UNSUPPORTED) {
            rc = lin(w.h, H, L(l, MINITP_W_GATE_UP), nullptr, w.gu, 2 * I, 2 * I, H);
            const char* up = (const char*)w.gu + I * es();
            if (!rc) rc = launch_silu_mul(st, c.dtype, w.gu, up, 2 * I, w.act, I, M, I);
          }
          if (rc) return rc;
        }
        // x += down(act), h = the next layer's input_layernorm(x) (the final norm after the last)
        const void* next_norm = l + 1 < c.num_layers ? L(l + 1, MINITP_W_LN1) : final_norm;
        // (a long K over too few tiles, e.g. 7B at 512 tokens: the tile kernel
        // with every tile split over K, then the residual add + norm)
        if (MINITP_DOWN_TILE_SPLIT && gemm_tile_split_supported(M, H, I, I, H, false)) {
          rc = launch_gemm_tile_split(st, w.act, I, L(l, MINITP_W_DOWN), nullptr, w.h, H, M, H, I, false, tail);
          if (!rc) rc = launch_add_rmsnorm(st, c.dtype, w.x, w.h, next_norm, w.h, M, H, c.eps);
          if (rc) return rc;
          continue;
        }
        rc = partials(w.act, I, L(l, MINITP_W_DOWN), H, I, &pp);
        if (rc == MINITP_OK) {
          rc = launch_add_rmsnorm_partials(st, w.x, pp, next_norm, w.h, H, c.eps);
        } else if (rc == MINITP_ERR_UNSUPPORTED) {
          rc = lin(w.act, I, L(l, MINITP_W_DOWN), nullptr, w.h, H, H, I);
          if (!rc) rc = launch_add_rmsnorm(st, c.dtype, w.x, w.h, next_norm, w.h, M, H, c.eps);
        }
        if (rc) return rc;
        continue;
      }
      // ---- attention block --------------------------------------------------
      if (fz) {
        GemvArgs g{};
        g.x = w.x;
        g.ldx = H;
        g.norm_w = L(l, MINITP_W_LN1);
        g.eps = c.eps;
        g.w = L(l, MINITP_W_QKV);
        g.bias = L(l, MINITP_W_QKV_BIAS);
        g.y = w.q;
        g.ldy = q_rows();
        g.M = M;
        g.N = qkv_rows();
        g.K = H;
        g.st = w.st;
        g.cos_tab = cos_tab;
        g.sin_tab = sin_tab;
        g.max_pos = c.max_pos;
        g.layer = l;
        g.a = as;
        if ((rc = launch_gemv(st, c.dtype, PRO_NORM, EPI_QKV_ROPE, g))) return rc;
      } else {
        if ((rc = launch_rmsnorm(st, c.dtype, w.x, L(l, MINITP_W_LN1), w.h, M, H, c.eps))) return rc;
        if ((rc = launch_gemm(st, c.dtype, w.h, H, L(l, MINITP_W_QKV), L(l, MINITP_W_QKV_BIAS), w.qkv, qkv_rows(), M,
                              qkv_rows(), H, MINITP_EPI_NONE, nullptr, nullptr, w.gemm_ws, GEMM_SPLIT_BYTES)))
          return rc;
        if ((rc = launch_rope_kv_write(st, c.dtype, w.qkv, qkv_rows(), w.q, nullptr, nullptr, cos_tab, sin_tab, nullptr,
                                       c.max_pos, B, T, c.heads, c.kv_heads, D, s.max_seq, 0, nullptr, w.st, l)))
          return rc;
      }
      if (fo) {
        const OprojArgs o{L(l, MINITP_W_O), H, attn_oproj_rows(c.dtype, as, H, OPROJ_SLICES), w.opart};
        if ((rc = launch_decode_attention_oproj(st, c.dtype, w.q, as, w.st, l, o))) return rc;
      } else if (T == 1) {
        if ((rc = launch_decode_attention(st, c.dtype, w.q, nullptr, nullptr, w.attn, as, s.cache_len, w.st, l,
                                          w.attn_ws, w.attn_ws_bytes)))
          return rc;
      } else {
        const char* kc = (const char*)s.k_cache + l * layer_elems * es();
        const char* vc = (const char*)s.v_cache + l * layer_elems * es();
        if ((rc = launch_prefill_attention(st, c.dtype, w.q, kc, vc, w.attn, as, s.cache_len, w.st, l))) return rc;
      }
      if (fo) {
        // (o_proj ran in the attention kernel)
      } else if (fz) {
        GemvArgs g{};
        g.x = w.attn;
        g.ldx = q_rows();
        g.w = L(l, MINITP_W_O);
        g.y = w.x;
        g.ldy = H;
        g.aux = w.x;
        g.M = M;
        g.N = H;
        g.K = q_rows();
        // (MFMA rows: the unsplit MFMA form; its one round trip beats the
        // split form's three extra at K = 896)
        if (!gemv_mfma_rows(c.dtype, M)) split_bufs(g);
        if ((rc = launch_gemv(st, c.dtype, PRO_NONE, EPI_RESID, g))) return rc;
      } else {
        if ((rc = launch_gemm(st, c.dtype, w.attn, q_rows(), L(l, MINITP_W_O), nullptr, w.x, H, M, H, q_rows(),
                              MINITP_EPI_RESID, w.x, nullptr, w.gemm_ws, GEMM_SPLIT_BYTES)))
          return rc;
      }
      // ---- MLP block ----------------------------------------------------------
      if (fz) {
        GemvArgs g{};
        g.x = w.x;
        g.ldx = H;
        g.norm_w = L(l, MINITP_W_LN2);
        g.eps = c.eps;
        g.w = L(l, MINITP_W_GATE_UP);
        g.y = w.act;
        g.ldy = I;
        g.M = M;
        g.N = I;
        g.K = H;
        if (fo) {
          // x + o_proj (the attention's partials) -> h, then as above
          g.part = w.opart;
          g.nparts = c.heads;
          g.x_out = w.h;
          if ((rc = launch_gemv_part_swiglu(st, c.dtype, g))) return rc;
        } else if ((rc = launch_gemv(st, c.dtype, PRO_NORM, EPI_SWIGLU, g))) {
          return rc;
        }
        // the down projection's long K splits over blocks (register form
        // past 8,192, MFMA form at 5..32 rows)
        GemvArgs d{};
        d.x = w.act;
        d.ldx = I;
        d.w = L(l, MINITP_W_DOWN);
        d.y = w.x;
        d.ldy = H;
        d.aux = fo ? w.h : w.x;
        d.M = M;
        d.N = H;
        d.K = I;
        split_bufs(d);
        if ((rc = launch_gemv(st, c.dtype, PRO_NONE, EPI_RESID, d))) return rc;
      } else {
        if ((rc = launch_rmsnorm(st, c.dtype, w.x, L(l, MINITP_W_LN2), w.h, M, H, c.eps))) return rc;
        if ((rc = launch_gemm(st, c.dtype, w.h, H, L(l, MINITP_W_GATE_UP), nullptr, w.gu, 2 * I, M, 2 * I, H,
                              MINITP_EPI_NONE, nullptr, nullptr, w.gemm_ws, GEMM_SPLIT_BYTES)))
          return rc;
        const char* up = (const char*)w.gu + I * es();
        if ((rc = launch_silu_mul(st, c.dtype, w.gu, up, 2 * I, w.act, I, M, I))) return rc;
        if ((rc = launch_gemm(st, c.dtype, w.act, I, L(l, MINITP_W_DOWN), nullptr, w.x, H, M, H, I, MINITP_EPI_RESID,
                              w.x, nullptr, w.gemm_ws, GEMM_SPLIT_BYTES)))
          return rc;
      }
    }
    // ---- final norm, LM head, greedy pick ----------------------------------------
    if (!s.logits_all && gemv_supported(c.dtype, B, H) && !gemv_mfma_rows(c.dtype, B)) {
      GemvArgs g{};
      g.x = (const char*)w.x + (T - 1) * H * es();  // last position of each row
      g.ldx = T * H;
      g.norm_w = final_norm;
      g.eps = c.eps;
      g.w = lm_head;
      g.M = B;
      g.N = V;
      g.K = H;
      g.st = w.st;
      g.part_val = w.part_val;
      g.part_idx = w.part_idx;
      return launch_gemv(st, c.dtype, PRO_NORM, EPI_ARGMAX, g);
    }
    if (!s.logits_all && gemv_mfma_rows(c.dtype, B) && gemv_norm_supported(c.dtype, B, H)) {
      // batched rows (bf16 MFMA rows): the final norm and the LM head in one
      // MFMA GEMV whose blocks each normalize the rows once for many tuples,
      // storing the step's logits (read from the step state), then the argmax
      GemvArgs g{};
      g.x = (const char*)w.x + (T - 1) * H * es();
      g.ldx = T * H;
      g.norm_w = final_norm;
      g.eps = c.eps;
      g.w = lm_head;
      g.ldy = V;
      g.M = B;
      g.N = V;
      g.K = H;
      g.st = w.st;
      if ((rc = launch_gemv(st, c.dtype, PRO_NORM, EPI_STORE, g))) return rc;
      if (s.next_tok) return launch_argmax(st, c.dtype, nullptr, V, B, V, nullptr, 0, w.amax_ws, w.amax_ws_bytes, w.st, 0);
      return MINITP_OK;
    }
    if (s.logits_all && fz) {  // same kernel family as the module path at this M
      GemvArgs g{};
      g.x = w.x;
      g.ldx = H;
      g.norm_w = final_norm;
      g.eps = c.eps;
      g.w = lm_head;
      g.y = s.logits;  // (not captured: prompt_graphable)
      g.ldy = V;
      g.M = M;
      g.N = V;
      g.K = H;
      if ((rc = launch_gemv(st, c.dtype, PRO_NORM, EPI_STORE, g))) return rc;
      if (s.next_tok)
        return launch_argmax(st, c.dtype, nullptr, T * V, B, V, nullptr, 0, w.amax_ws, w.amax_ws_bytes, w.st,
                             (T - 1) * V);
      return MINITP_OK;
    }
    if (!blas && (rc = launch_rmsnorm(st, c.dtype, w.x, final_norm, w.h, M, H, c.eps))) return rc;
    if (s.logits_all) {  // (with blas, h already holds norm(x))
      rc = MINITP_ERR_UNSUPPORTED;
      if (blas && gemm_tile_supported(M, V, H, H, V, false))
        rc = launch_gemm_tile(st, w.h, H, lm_head, nullptr, s.logits, V, M, V, H, false, tail);
      if (rc == MINITP_ERR_UNSUPPORTED)
        rc = launch_gemm(st, c.dtype, w.h, H, lm_head, nullptr, nullptr, V, M, V, H, MINITP_EPI_NONE, nullptr, w.st);
      if (rc) return rc;
      if (s.next_tok)
        return launch_argmax(st, c.dtype, nullptr, T * V, B, V, nullptr, 0, w.amax_ws, w.amax_ws_bytes, w.st,
                             (T - 1) * V);
      return MINITP_OK;
    }
    const char* hl = (const char*)w.h + (T - 1) * H * es();
    if ((rc = launch_gemm(st, c.dtype, hl, T * H, lm_head, nullptr, nullptr, V, B, V, H, MINITP_EPI_NONE, nullptr,
                          w.st)))
      return rc;
    if (s.next_tok) return launch_argmax(st, c.dtype, nullptr, V, B, V, nullptr, 0, w.amax_ws, w.amax_ws_bytes, w.st, 0);
    return MINITP_OK;
  }

  int check_step(const minitp_qwen2_step* s, Ws& w) {
    MINITP_CHECK_ARG(s != nullptr, "step is NULL");
    MINITP_CHECK_ARG(s->batch >= 1 && s->tokens >= 1, "batch=%lld tokens=%lld", (long long)s->batch,
                     (long long)s->tokens);
    MINITP_CHECK_ARG(s->ids && s->positions && s->k_cache && s->v_cache && s->workspace, "NULL pointer in step");
    MINITP_CHECK_ARG(s->logits != nullptr || s->next_tok != nullptr, "step produces nothing (no logits, no next_tok)");
    // Only the fused LM-head GEMV + argmax (last position, batch <= 4) can
    // skip the logits store; the other LM-head paths always write them.
    const bool fused_head = !s->logits_all && s->batch <= 4 && gemv_supported(c.dtype, s->batch, c.hidden);
    MINITP_CHECK_ARG(fused_head || s->logits != nullptr,
                     "logits buffer required (batch %lld, logits_all %d: the LM head stores logits before the argmax)",
                     (long long)s->batch, (int)s->logits_all);
    MINITP_CHECK_ARG(s->ids_ld >= s->tokens, "ids_ld=%lld < tokens", (long long)s->ids_ld);
    MINITP_CHECK_ARG(s->eos_state == nullptr || (s->next_tok != nullptr && s->eos_token >= 0 && s->cursor >= 0),
                     "early stop needs next_tok, eos_token >= 0 and cursor >= 0 (eos_token %lld, cursor %lld)",
                     (long long)s->eos_token, (long long)s->cursor);
    if (s->cache_len < 0 || s->cache_len + s->tokens > s->max_seq) {
      set_error("KV cache overflow: seq %lld+%lld > max_seq_len=%lld", (long long)s->cache_len, (long long)s->tokens,
                (long long)s->max_seq);
      return MINITP_ERR_OVERFLOW;
    }
    const int64_t M = s->batch * s->tokens;
    w = layout(s->workspace, M, s->batch, s->max_seq);
    if (s->workspace_bytes < w.bytes) {
      set_error("workspace %lld B < %lld B needed for %lld rows, batch %lld, max_seq %lld",
                (long long)s->workspace_bytes, (long long)w.bytes, (long long)M, (long long)s->batch,
                (long long)s->max_seq);
      return MINITP_ERR_ARG;
    }
    return MINITP_OK;
  }

  ~Qwen2Program() {
    for (auto& g : graphs) {
      (void)hipGraphExecDestroy(g.exec);
      (void)hipGraphDestroy(g.graph);
    }
    if (capture_stream) (void)hipStreamDestroy(capture_stream);
  }
};

static int patch_and_launch(Qwen2Program* p, GraphEntry& g, hipStream_t st, const minitp_qwen2_step& s, const Ws& w) {
  StepArgs val = step_args(s);
  StepState* dst = w.st;
  const void* table = p->embed;
  void* out = w.x;
  int64_t hidden = p->c.hidden, vocab = p->c.vocab, tt = s.tokens, max_pos = p->c.max_pos;
  const float* cos_tab = p->cos_tab;
  const float* sin_tab = p->sin_tab;
  int head_dim = p->c.head_dim;
  void* args[] = {&dst, &val, (void*)&table, &out, &hidden, &vocab, &tt, (void*)&cos_tab, (void*)&sin_tab,
                  &max_pos, &head_dim};
  hipKernelNodeParams kp{};
  kp.func = p->c.dtype == MINITP_F32 ? (void*)step_embed_kernel<float> : (void*)step_embed_kernel<bf16>;
  kp.gridDim = dim3((unsigned)(s.batch * s.tokens));
  kp.blockDim = dim3(EMBED_THREADS);
  kp.sharedMemBytes = 0;
  kp.kernelParams = args;
  kp.extra = nullptr;
  MINITP_RETURN_HIP(hipGraphExecKernelNodeSetParams(g.exec, g.first, &kp));
  MINITP_RETURN_HIP(hipGraphLaunch(g.exec, st));
  return MINITP_OK;
}

// One forward through a captured graph of its launch sequence: replayed when
// a graph of this shape (batch, tokens, max_seq, workspace, early stop, token
// pick, all-position logits: everything the launch sequence depends on)
// exists, else run eagerly once and recorded. Every kernel after the
// first reads the per-call values (ids, positions, cache_len, caches, logits,
// token outputs) from the step state the first kernel writes, so only that
// kernel's parameters are patched per call.
static int run_graphed(Qwen2Program* p, hipStream_t st, const minitp_qwen2_step& s, const Ws& w) {
  // a caller capturing its own stream records the direct launch sequence
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) return p->run(st, s, w);
  std::lock_guard<std::mutex> lock(p->mu);
  const GraphKey key{s.batch, s.tokens, s.max_seq, s.workspace, s.eos_state != nullptr, s.next_tok != nullptr,
                     s.logits_all != 0};
  const uint64_t now = ++p->clock;
  // calls of this shape
  ShapeCalls* sc = nullptr;
  for (auto& c : p->shape_calls)
    if (c.key == key) sc = &c;
  if (sc == nullptr) {
    if (p->shape_calls.size() >= 64) {  // forget the shape called least recently
      auto old = p->shape_calls.begin();
      for (auto it = p->shape_calls.begin(); it != p->shape_calls.end(); ++it)
        if (it->last < old->last) old = it;
      p->shape_calls.erase(old);
    }
    p->shape_calls.push_back(ShapeCalls{key, 0, 0});
    sc = &p->shape_calls.back();
  }
  ++sc->calls;
  sc->last = now;
  const uint64_t calls = sc->calls;
  for (auto& g : p->graphs)
    if (g.key == key) {
      g.last_use = now;
      g.last_stream = st;
      return patch_and_launch(p, g, st, s, w);
    }
  // Not recorded: run directly. A prompt shape is recorded on its second
  // call (a one-off prompt length pays no capture), a decode shape on its
  // first. When the cache already holds 8 graphs of this kind, the shape
  // takes the place of the least recently used one only if it has been
  // called more often than that one, so a rotation of more shapes than the
  // cache holds settles on replaying 8 of them instead of re-recording.
  int rc = p->run(st, s, w);
  if (rc) return rc;
  const bool prompt = s.tokens > 1;
  if (prompt && calls < 2) return MINITP_OK;
  GraphEntry* victim = nullptr;
  int same_kind = 0;
  for (auto& e : p->graphs)
    if ((e.key.tokens > 1) == prompt) {
      ++same_kind;
      if (victim == nullptr || e.last_use < victim->last_use) victim = &e;
    }
  if (same_kind >= 8) {
    uint64_t victim_calls = 0;
    for (const auto& c : p->shape_calls)
      if (c.key == victim->key) victim_calls = c.calls;
    if (calls <= victim_calls) return MINITP_OK;
  }
  if (!p->capture_stream) MINITP_RETURN_HIP(hipStreamCreateWithFlags(&p->capture_stream, hipStreamNonBlocking));
  GraphEntry g{};
  g.key = key;
  g.last_use = now;
  g.last_stream = st;
  MINITP_RETURN_HIP(hipStreamBeginCapture(p->capture_stream, hipStreamCaptureModeRelaxed));
  rc = p->run(p->capture_stream, s, w);
  hipError_t e = hipStreamEndCapture(p->capture_stream, &g.graph);
  if (rc) {
    if (e == hipSuccess) (void)hipGraphDestroy(g.graph);
    return rc;
  }
  MINITP_RETURN_HIP(e);
  size_t n_roots = 0;
  MINITP_RETURN_HIP(hipGraphGetRootNodes(g.graph, nullptr, &n_roots));
  if (n_roots != 1) {
    (void)hipGraphDestroy(g.graph);
    set_error("forward graph has %zu root nodes, expected 1", n_roots);
    return MINITP_ERR_HIP;
  }
  MINITP_RETURN_HIP(hipGraphGetRootNodes(g.graph, &g.first, &n_roots));
  MINITP_RETURN_HIP(hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0));
  if (same_kind >= 8) {
    // a replay of the victim may still be running: wait for the stream it
    // was last launched on before destroying it
    (void)hipStreamSynchronize(victim->last_stream);
    (void)hipGraphExecDestroy(victim->exec);
    (void)hipGraphDestroy(victim->graph);
    p->graphs.erase(p->graphs.begin() + (victim - p->graphs.data()));
  }
  p->graphs.push_back(g);
  return MINITP_OK;
}

}  // namespace minitp

using minitp::Qwen2Program;

extern "C" {

int minitp_qwen2_create(const minitp_qwen2_config* cfg, const minitp_qwen2_weights* w, void** handle) {
  MINITP_CHECK_ARG(cfg && w && handle, "NULL argument");
  const auto& c = *cfg;
  MINITP_CHECK_ARG(c.dtype == MINITP_F32 || c.dtype == MINITP_BF16, "dtype %d", c.dtype);
  MINITP_CHECK_ARG(c.num_layers > 0 && c.hidden > 0 && c.heads > 0 && c.kv_heads > 0 && c.head_dim > 0 &&
                       c.intermediate > 0 && c.vocab > 0 && c.max_pos > 0,
                   "non-positive dimension in config");
  MINITP_CHECK_ARG(c.heads % c.kv_heads == 0, "num_attention_heads=%d not divisible by num_key_value_heads=%d",
                   c.heads, c.kv_heads);
  MINITP_CHECK_ARG(c.head_dim % 8 == 0 && c.hidden % 8 == 0 && c.intermediate % 8 == 0,
                   "hidden, intermediate and head_dim must be multiples of 8");
  MINITP_CHECK_ARG(w->embed && w->lm_head && w->final_norm && w->rope_cos && w->rope_sin && w->layers,
                   "NULL weight pointer");
  for (int i = 0; i < c.num_layers * MINITP_W_PER_LAYER; ++i)
    MINITP_CHECK_ARG(w->layers[i] != nullptr && minitp::aligned16(w->layers[i]), "layer weight %d NULL or unaligned",
                     i);
  auto* p = new (std::nothrow) Qwen2Program();
  if (p != nullptr) {
    const char* pg = getenv("MINITP_PREFILL_GRAPH");
    p->prefill_graphs = !(pg != nullptr && pg[0] == '0');
    const char* fo = getenv("MINITP_FUSE_OPROJ");
    p->fuse_oproj = !(fo != nullptr && fo[0] == '0');
  }
  if (!p) {
    minitp::set_error("out of host memory");
    return MINITP_ERR_HIP;
  }
  p->c = c;
  p->embed = w->embed;
  p->lm_head = w->lm_head;
  p->final_norm = w->final_norm;
  p->cos_tab = w->rope_cos;
  p->sin_tab = w->rope_sin;
  p->lw.assign(w->layers, w->layers + (size_t)c.num_layers * MINITP_W_PER_LAYER);
  *handle = p;
  return MINITP_OK;
}

int minitp_qwen2_decode_check(void* handle, void* stream, void* workspace) {
  MINITP_CHECK_ARG(handle != nullptr && workspace != nullptr, "NULL argument");
  MINITP_RETURN_HIP(hipStreamSynchronize((hipStream_t)stream));
  // the step state sits at the start of every workspace (layout())
  auto* state = (minitp::StepState*)workspace;
  int32_t err = 0;
  MINITP_RETURN_HIP(hipMemcpy(&err, &state->error, sizeof(err), hipMemcpyDeviceToHost));
  if (err == 0) return MINITP_OK;
  const int32_t zero = 0;
  MINITP_RETURN_HIP(hipMemcpy(&state->error, &zero, sizeof(zero), hipMemcpyHostToDevice));
  minitp::set_error("position out of range for the RoPE table of %d rows (a forward on this workspace ran with NaN "
                    "rotary rows)",
                    ((Qwen2Program*)handle)->c.max_pos);
  return MINITP_ERR_RANGE;
}

int minitp_qwen2_destroy(void* handle) {
  delete (Qwen2Program*)handle;
  return MINITP_OK;
}

int64_t minitp_qwen2_workspace_bytes(void* handle, int64_t max_tokens, int64_t batch, int64_t max_seq) {
  if (!handle || max_tokens < 1 || batch < 1 || max_seq < 1) return -1;
  return ((Qwen2Program*)handle)->layout(nullptr, max_tokens, batch, max_seq).bytes;
}

int minitp_qwen2_forward(void* handle, void* stream, const minitp_qwen2_step* step) {
  MINITP_CHECK_ARG(handle != nullptr, "NULL handle");
  auto* p = (Qwen2Program*)handle;
  minitp::Ws w;
  int rc = p->check_step(step, w);
  if (rc) return rc;
  if (p->prompt_graphable(*step)) return minitp::run_graphed(p, (hipStream_t)stream, *step, w);
  return p->run((hipStream_t)stream, *step, w);
}

int minitp_qwen2_decode(void* handle, void* stream, const minitp_qwen2_step* step_in) {
  MINITP_CHECK_ARG(handle != nullptr && step_in != nullptr, "NULL argument");
  auto* p = (Qwen2Program*)handle;
  MINITP_CHECK_ARG(step_in->tokens == 1, "decode expects tokens == 1, got %lld", (long long)step_in->tokens);
  // With one token, [B, T, V] and [B, V] logits are the same layout: one
  // graph shape serves both (and no logits pointer is baked into a graph).
  minitp_qwen2_step one = *step_in;
  one.logits_all = 0;
  const minitp_qwen2_step* step = &one;
  minitp::Ws w;
  int rc = p->check_step(step, w);
  if (rc) return rc;
  return minitp::run_graphed(p, (hipStream_t)stream, *step, w);
}

}  // extern "C"
