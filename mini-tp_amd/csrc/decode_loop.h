// Persistent batch-1 decode (decode_loop.hip): parameters shared by the
// kernel and the host-side program.
#pragma once

#include "common.h"

namespace minitp {

constexpr int LOOP_MAX_BLOCKS = 1024;
constexpr int LOOP_THREADS = 512;
constexpr int LOOP_CTRL_BYTES = 256;
// 32-bit control words at the start of the persistent region of a workspace
enum { LOOP_CTRL_EPOCH = 0, LOOP_CTRL_ERROR = 1, LOOP_CTRL_ABORT = 2 };
enum { LOOP_ERR_TIMEOUT = 1, LOOP_ERR_POSITION = 2 };

// One layer's weights, as the device-side table holds them.
struct LoopLayerW {
  const void* ln1;
  const void* ln2;
  const void* wqkv;
  const void* bqkv;
  const void* wo;
  const void* wgu;
  const void* wdown;
  const void* pad;
};

// LL words (8 bytes each) of the persistent region: per layer the q/k/v pair
// words, the per-group o_proj partials, the SwiGLU activations and the down
// outputs; after the layers, two words per block of LM-head argmax partials.
struct LoopLayout {
  int64_t off_qkv, off_p, off_act, off_down, layer_words, off_lm, total_words, bytes;
};

// Byte offsets of the kernel's dynamic LDS.
struct LoopLds {
  int xs, xin, stage, qstage, rowres, norm, tile, misc, bytes;
};

struct LoopParams {
  int L, H, Hq, Hkv, G, I, V;
  float eps, scale;
  int64_t S, max_pos;
  const void* embed;
  const void* lm_head;
  const void* final_norm;
  const float* cos_tab;
  const float* sin_tab;
  const LoopLayerW* layers;
  const int64_t* ids;
  const int64_t* positions;
  int64_t cache_len;
  void* k_cache;
  void* v_cache;
  void* logits;
  int64_t* next_tok;
  uint32_t* ctrl;
  uint64_t* ll;
  int64_t ll_layer_words, off_qkv, off_p, off_act, off_down, off_lm;
  int lds_xs, lds_xin, lds_stage, lds_qstage, lds_rowres, lds_norm, lds_tile, lds_misc;
  int64_t spin_limit;  // wall-clock ticks a wait may last
  // Wave roles: waves [role[0], role[1]) stream the QKV weights, [role[1],
  // role[2]) o_proj (and copy K / V tiles), [role[2], role[3]) gate/up,
  // [role[3], role[4]) down; role[0] == 1, role[4] == LOOP_THREADS / 64.
  int role[5];
  // Optional phase trace: when non-null, lane 0 of wave w of block b writes
  // the wall clock at every phase point to trace[(b * trace_slots + slot) *
  // (LOOP_THREADS / 64) + w].
  uint64_t* trace;
  int trace_slots;
};

// Trace slots: LOOP_TRACE_START, then LOOP_TRACE_PER_LAYER per layer, then
// the LM head's.
enum {
  LOOP_TR_START = 0,
  LOOP_TR_A_IN = 0, LOOP_TR_A_OUT, LOOP_TR_A_ISSUED, LOOP_TR_B_IN, LOOP_TR_B_ATTN, LOOP_TR_B_OUT, LOOP_TR_B_ISSUED,
  LOOP_TR_C_IN, LOOP_TR_C_OUT, LOOP_TR_C_ISSUED, LOOP_TR_D_IN, LOOP_TR_D_OUT, LOOP_TR_D_ISSUED, LOOP_TR_ATT_SC,
  LOOP_TR_ATT_PV, LOOP_TR_PER_LAYER
};
inline int loop_trace_slots(int layers) { return 1 + layers * LOOP_TR_PER_LAYER + 4; }

LoopLayout loop_layout(const minitp_qwen2_config& c);
const char* loop_unsupported(const minitp_qwen2_config& c, int nb, LoopLds* out);
const void* loop_kernel(int dtype, int D);
void loop_roles(const minitp_qwen2_config& c, int nb, int* out);

}  // namespace minitp
