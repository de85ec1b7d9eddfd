// extern "C" entry points of include/minitp.h: validate on the host, then
// launch. Nothing here allocates, synchronises or throws.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <unordered_map>

#include "common.h"
#include "kernels.h"

namespace minitp {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

}  // namespace minitp

using namespace minitp;

namespace {

inline hipStream_t S(void* s) { return (hipStream_t)s; }
inline bool dtype_ok(int d) { return d == MINITP_F32 || d == MINITP_BF16; }
inline int vec_elems(int dtype) { return dtype == MINITP_F32 ? 4 : 8; }

#define CHECK_DTYPE(d) MINITP_CHECK_ARG(dtype_ok(d), "dtype %d is not MINITP_F32 or MINITP_BF16", (int)(d))

}  // namespace

extern "C" {

const char* minitp_status_string(int status) {
  switch (status) {
    case MINITP_OK:
      return "ok";
    case MINITP_ERR_ARG:
      return "invalid argument";
    case MINITP_ERR_HIP:
      return "HIP runtime error";
    case MINITP_ERR_OVERFLOW:
      return "KV cache overflow";
    case MINITP_ERR_RANGE:
      return "index out of range";
    case MINITP_ERR_UNSUPPORTED:
      return "unsupported";
    case MINITP_ERR_DIVISIBLE:
      return "not divisible";
  }
  return "unknown status";
}

const char* minitp_last_error(void) { return g_err; }

int minitp_abi_version(void) { return MINITP_ABI_VERSION; }

int minitp_fill_normal(void* stream, int dtype, void* dst, int64_t count, uint64_t seed, uint64_t stream_id,
                       double std_dev) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(count >= 0 && (count == 0 || dst), "fill_normal: count=%lld dst=%p", (long long)count, dst);
  if (count == 0) return MINITP_OK;
  return launch_fill_normal(S(stream), dtype, dst, count, seed, stream_id, std_dev);
}

int minitp_fill_uniform_ids(void* stream, int64_t* dst, int64_t count, uint64_t seed, uint64_t stream_id,
                            int64_t vocab) {
  MINITP_CHECK_ARG(count >= 0 && (count == 0 || dst) && vocab > 0 && vocab < (1LL << 32),
                   "fill_uniform_ids: count=%lld vocab=%lld", (long long)count, (long long)vocab);
  if (count == 0) return MINITP_OK;
  return launch_fill_ids(S(stream), dst, count, seed, stream_id, vocab);
}

int minitp_fill(void* stream, int dtype, void* dst, int64_t count, float value) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(count >= 0 && (count == 0 || dst), "fill: count=%lld", (long long)count);
  if (count == 0) return MINITP_OK;
  return launch_fill(S(stream), dtype, dst, count, value);
}

int minitp_embedding(void* stream, int dtype, const void* table, const int64_t* ids, void* out, int64_t n_tokens,
                     int64_t hidden, int64_t vocab) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(n_tokens >= 0 && hidden > 0 && vocab > 0, "embedding: n=%lld hidden=%lld vocab=%lld",
                   (long long)n_tokens, (long long)hidden, (long long)vocab);
  if (n_tokens == 0) return MINITP_OK;
  MINITP_CHECK_ARG(table && ids && out, "embedding: NULL pointer");
  MINITP_CHECK_ARG(hidden % vec_elems(dtype) == 0 && aligned16(table) && aligned16(out),
                   "embedding: hidden must be a multiple of 16 bytes and pointers 16-byte aligned");
  return launch_embedding(S(stream), dtype, table, ids, 1, n_tokens, 1, out, hidden, vocab);
}

int minitp_rmsnorm(void* stream, int dtype, const void* x, const void* w, void* out, int64_t rows, int64_t hidden,
                   float eps) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(rows >= 0 && hidden > 0, "rmsnorm: rows=%lld hidden=%lld", (long long)rows, (long long)hidden);
  if (rows == 0) return MINITP_OK;
  MINITP_CHECK_ARG(x && w && out, "rmsnorm: NULL pointer");
  return launch_rmsnorm(S(stream), dtype, x, w, out, rows, hidden, eps);
}

int minitp_add(void* stream, int dtype, const void* a, const void* b, void* out, int64_t n, int64_t b_period) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(n >= 0 && (n == 0 || (a && b && out)), "add: n=%lld", (long long)n);
  MINITP_CHECK_ARG(b_period > 0 && n % b_period == 0, "add: b_period=%lld must divide n=%lld", (long long)b_period,
                   (long long)n);
  return launch_add(S(stream), dtype, a, b, out, n, b_period);
}

int minitp_silu_mul(void* stream, int dtype, const void* gate, const void* up, int64_t ld_in, void* out,
                    int64_t ld_out, int64_t rows, int64_t n) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(rows >= 0 && n >= 0 && ld_in >= n && ld_out >= n, "silu_mul: rows=%lld n=%lld ld=%lld/%lld",
                   (long long)rows, (long long)n, (long long)ld_in, (long long)ld_out);
  if (rows * n == 0) return MINITP_OK;
  MINITP_CHECK_ARG(gate && up && out, "silu_mul: NULL pointer");
  return launch_silu_mul(S(stream), dtype, gate, up, ld_in, out, ld_out, rows, n);
}

int minitp_host_device_pointer(void* host, void** device) {
  MINITP_CHECK_ARG(host != nullptr && device != nullptr, "NULL pointer");
  MINITP_RETURN_HIP(hipHostGetDevicePointer(device, host, 0));
  return MINITP_OK;
}

int minitp_cast_f32_bf16(void* stream, const float* in, void* out, int64_t n) {
  MINITP_CHECK_ARG(n >= 0, "cast: n=%lld", (long long)n);
  if (n == 0) return MINITP_OK;
  MINITP_CHECK_ARG(in && out, "cast: NULL pointer");
  return launch_cast_f32_bf16(S(stream), in, out, n);
}

namespace {

int linear_checks(int dtype, const void* x, int64_t ldx, const void* w, const void* bias, void* y, int64_t ldy,
                  int64_t M, int64_t N, int64_t K, int epilogue, const void* aux) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(M >= 0 && N >= 0 && K > 0, "linear: M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                   (long long)K);
  MINITP_CHECK_ARG(epilogue >= MINITP_EPI_NONE && epilogue <= MINITP_EPI_SWIGLU, "linear: epilogue %d", epilogue);
  if (M == 0 || N == 0) return MINITP_OK;
  MINITP_CHECK_ARG(x && w && y, "linear: NULL pointer");
  MINITP_CHECK_ARG(K % vec_elems(dtype) == 0, "linear: K=%lld must be a multiple of %d", (long long)K,
                   vec_elems(dtype));
  MINITP_CHECK_ARG(ldx >= K && ldy >= N && ldx % vec_elems(dtype) == 0, "linear: ldx=%lld ldy=%lld",
                   (long long)ldx, (long long)ldy);
  MINITP_CHECK_ARG(aligned16(x) && aligned16(w), "linear: x and W must be 16-byte aligned");
  MINITP_CHECK_ARG(epilogue != MINITP_EPI_RESID || aux != nullptr, "linear: RESID needs aux");
  MINITP_CHECK_ARG(epilogue == MINITP_EPI_NONE || bias == nullptr, "linear: bias only with MINITP_EPI_NONE");
  if (epilogue == MINITP_EPI_SWIGLU)
    MINITP_CHECK_ARG(N % 2 == 0, "linear: SWIGLU output width %lld must be even", (long long)N);
  return MINITP_OK;
}

GemvArgs gemv_args(const void* x, int64_t ldx, const void* w, const void* bias, void* y, int64_t ldy, int64_t M,
                   int64_t N, int64_t K, const void* aux) {
  GemvArgs g{};
  g.x = x;
  g.ldx = ldx;
  g.w = w;
  g.bias = bias;
  g.y = y;
  g.ldy = ldy;
  g.aux = aux;
  g.M = M;
  g.N = N;
  g.K = K;
  return g;
}

int gemv_epilogue(int epilogue) {
  return epilogue == MINITP_EPI_RESID ? EPI_RESID : epilogue == MINITP_EPI_SWIGLU ? EPI_SWIGLU : EPI_STORE;
}

}  // namespace

int minitp_linear(void* stream, int dtype, const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                  int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue, const void* aux) {
  int rc = linear_checks(dtype, x, ldx, w, bias, y, ldy, M, N, K, epilogue, aux);
  if (rc || M == 0 || N == 0) return rc;
  hipStream_t st = S(stream);
  if (gemv_supported(dtype, M, K))
    return launch_gemv(st, dtype, PRO_NONE, gemv_epilogue(epilogue), gemv_args(x, ldx, w, bias, y, ldy, M, N, K, aux));
  if (epilogue == MINITP_EPI_SWIGLU) {
    if (dtype == MINITP_BF16 && bias == nullptr && aligned16(x) && aligned16(w) &&
        gemm_tile_supported(M, N, K, ldx, ldy, true))
      return launch_gemm_tile(st, x, ldx, w, nullptr, y, ldy, M, N, K, true);
    set_error("linear: SWIGLU epilogue is served for decode rows (M <= 4, bf16 up to 32) and bf16 prompts of at "
              "least 96 256 x 128 output tiles; use NONE + minitp_silu_mul");
    return MINITP_ERR_UNSUPPORTED;
  }
  return launch_gemm(st, dtype, x, ldx, w, bias, y, ldy, M, N, K, epilogue, aux);
}

int minitp_rmsnorm_linear(void* stream, int dtype, const void* x, int64_t ldx, const void* norm_w, float eps,
                          const void* w, const void* bias, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                          int epilogue, const void* aux) {
  int rc = linear_checks(dtype, x, ldx, w, bias, y, ldy, M, N, K, epilogue, aux);
  if (rc || M == 0 || N == 0) return rc;
  MINITP_CHECK_ARG(norm_w != nullptr, "rmsnorm_linear: NULL norm weight");
  MINITP_CHECK_ARG(epilogue != MINITP_EPI_RESID || aux != x, "rmsnorm_linear: RESID aux must not alias x");
  if (!gemv_norm_supported(dtype, M, K)) {
    set_error("rmsnorm_linear: M=%lld K=%lld is not a decode shape; use minitp_rmsnorm + minitp_linear",
              (long long)M, (long long)K);
    return MINITP_ERR_UNSUPPORTED;
  }
  GemvArgs g = gemv_args(x, ldx, w, bias, y, ldy, M, N, K, aux);
  g.norm_w = norm_w;
  g.eps = eps;
  return launch_gemv(S(stream), dtype, PRO_NORM, gemv_epilogue(epilogue), g);
}

int minitp_add_rmsnorm_linear_parts(void* stream, int dtype, const void* x, const float* parts, int32_t nparts,
                                    void* x_out, const void* norm_w, float eps, const void* w, void* y, int64_t N,
                                    int64_t K, int epilogue) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(x && parts && x_out && norm_w && w && y, "add_rmsnorm_linear_parts: NULL pointer");
  MINITP_CHECK_ARG(N >= 1 && K >= 1, "add_rmsnorm_linear_parts: N=%lld K=%lld", (long long)N, (long long)K);
  MINITP_CHECK_ARG(aligned16(x) && aligned16(parts) && aligned16(w) && aligned16(norm_w),
                   "add_rmsnorm_linear_parts: pointers must be 16-byte aligned");
  MINITP_CHECK_ARG(x_out != x, "add_rmsnorm_linear_parts: x_out must not alias x");
  if (epilogue != MINITP_EPI_SWIGLU || !gemv_part_supported(dtype, K, nparts)) {
    set_error("add_rmsnorm_linear_parts: serves the SwiGLU epilogue with K <= %lld (a multiple of 8 bf16 / 4 fp32) "
              "and 1..%d partial rows (epilogue %d, K %lld, %d rows)",
              (long long)PART_MAX_K, PART_MAX_PARTS, epilogue, (long long)K, (int)nparts);
    return MINITP_ERR_UNSUPPORTED;
  }
  GemvArgs g = gemv_args(x, K, w, nullptr, y, N, 1, N, K, nullptr);
  g.norm_w = norm_w;
  g.eps = eps;
  g.part = parts;
  g.nparts = nparts;
  g.x_out = x_out;
  return launch_gemv_part_swiglu(S(stream), dtype, g);
}

int minitp_rope(void* stream, int dtype, const void* q, const void* k, void* q_out, void* k_out, const float* cos_tab,
                const float* sin_tab, const int64_t* positions, int64_t B, int64_t Hq, int64_t Hkv, int64_t T,
                int64_t D) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(B >= 0 && Hq >= 0 && Hkv >= 0 && T >= 0 && D > 0 && D % 2 == 0, "rope: bad shape");
  if (B * T == 0) return MINITP_OK;
  MINITP_CHECK_ARG(q && k && q_out && k_out && cos_tab && sin_tab && positions, "rope: NULL pointer");
  return launch_rope(S(stream), dtype, q, k, q_out, k_out, cos_tab, sin_tab, positions, B, Hq, Hkv, T, D);
}

int minitp_kv_write(void* stream, int dtype, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                    int64_t B, int64_t H, int64_t T, int64_t D, int64_t S_, int64_t cache_len) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(B >= 0 && H >= 0 && T >= 0 && D > 0 && S_ >= 0 && cache_len >= 0, "kv_write: bad shape");
  if (cache_len + T > S_) {
    set_error("KV cache overflow: seq %lld+%lld > max_seq_len=%lld", (long long)cache_len, (long long)T,
              (long long)S_);
    return MINITP_ERR_OVERFLOW;
  }
  if (B * H * T == 0) return MINITP_OK;
  MINITP_CHECK_ARG(k_new && v_new && k_cache && v_cache, "kv_write: NULL pointer");
  return launch_kv_write(S(stream), dtype, k_new, v_new, k_cache, v_cache, B, H, T, D, S_, cache_len);
}

int minitp_rope_kv_write(void* stream, int dtype, const void* qkv, int64_t ld_qkv, void* q_out, void* k_cache,
                         void* v_cache, const float* cos_tab, const float* sin_tab, const int64_t* positions,
                         int64_t max_pos, int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t S_,
                         int64_t cache_len) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(B >= 0 && T >= 0 && Hq > 0 && Hkv > 0 && D > 0 && D % 2 == 0 && S_ >= 0 && cache_len >= 0,
                   "rope_kv_write: bad shape");
  MINITP_CHECK_ARG(ld_qkv >= (Hq + 2 * Hkv) * D, "rope_kv_write: ld_qkv=%lld", (long long)ld_qkv);
  if (cache_len + T > S_) {
    set_error("KV cache overflow: seq %lld+%lld > max_seq_len=%lld", (long long)cache_len, (long long)T,
              (long long)S_);
    return MINITP_ERR_OVERFLOW;
  }
  if (B * T == 0) return MINITP_OK;
  MINITP_CHECK_ARG(qkv && q_out && k_cache && v_cache && cos_tab && sin_tab && positions, "rope_kv_write: NULL");
  return launch_rope_kv_write(S(stream), dtype, qkv, ld_qkv, q_out, k_cache, v_cache, cos_tab, sin_tab, positions,
                              max_pos, B, T, Hq, Hkv, D, S_, cache_len, nullptr);
}

int64_t minitp_attention_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t S_) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || S_ < 0) return -1;
  return attention_workspace_bytes(B, T, Hq, Hkv, D, S_);
}

int minitp_attention(void* stream, int dtype, const void* q, const void* k_cache, const void* v_cache, void* out,
                     int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t S_, int64_t cache_len,
                     void* workspace, int64_t workspace_bytes) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(B >= 0 && T >= 0 && Hq > 0 && Hkv > 0 && D > 0 && cache_len >= 0, "attention: bad shape");
  if (Hq % Hkv != 0) {
    set_error("local q heads %lld not divisible by local kv heads %lld", (long long)Hq, (long long)Hkv);
    return MINITP_ERR_DIVISIBLE;
  }
  if (cache_len + T > S_) {
    set_error("KV cache overflow: seq %lld+%lld > max_seq_len=%lld", (long long)cache_len, (long long)T,
              (long long)S_);
    return MINITP_ERR_OVERFLOW;
  }
  if (B * T == 0) return MINITP_OK;
  MINITP_CHECK_ARG(q && k_cache && v_cache && out, "attention: NULL pointer");
  MINITP_CHECK_ARG(D % vec_elems(dtype) == 0 && aligned16(k_cache) && aligned16(v_cache),
                   "attention: head_dim rows must be 16-byte aligned");
  AttnShape a{(int)B, (int)T, (int)Hq, (int)Hkv, (int)D, S_};
  if (T == 1)
    return launch_decode_attention(S(stream), dtype, q, k_cache, v_cache, out, a, cache_len, nullptr, 0, workspace,
                                   workspace_bytes);
  return launch_prefill_attention(S(stream), dtype, q, k_cache, v_cache, out, a, cache_len);
}

int64_t minitp_argmax_workspace_bytes(int64_t B, int64_t V) {
  if (B < 0 || V <= 0) return -1;
  return argmax_workspace_bytes(B, V);
}

int minitp_argmax(void* stream, int dtype, const void* logits, int64_t ld, int64_t B, int64_t V, int64_t* out,
                  int64_t out_stride, void* workspace, int64_t workspace_bytes) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(B >= 0 && V > 0 && ld >= V, "argmax: B=%lld V=%lld ld=%lld", (long long)B, (long long)V,
                   (long long)ld);
  if (B == 0) return MINITP_OK;
  MINITP_CHECK_ARG(logits && out, "argmax: NULL pointer");
  return launch_argmax(S(stream), dtype, logits, ld, B, V, out, out_stride, workspace, workspace_bytes);
}

int64_t minitp_argmax_static_max_bytes(void) { return argmax_static_scratch_bytes(); }

int minitp_argmax_static(void* stream, int dtype, const void* logits, int64_t ld, int64_t B, int64_t V, int64_t* out,
                         int64_t out_stride) {
  CHECK_DTYPE(dtype);
  MINITP_CHECK_ARG(B >= 0 && V > 0 && ld >= V, "argmax_static: B=%lld V=%lld ld=%lld", (long long)B, (long long)V,
                   (long long)ld);
  if (B == 0) return MINITP_OK;
  MINITP_CHECK_ARG(logits && out, "argmax_static: NULL pointer");
  return launch_argmax_static(S(stream), dtype, logits, ld, B, V, out, out_stride);
}

}  // extern "C"

namespace minitp {

int ensure_lds_limit(const void* kernel, int bytes) {
  if (bytes <= 64 * 1024) return MINITP_OK;
  static std::mutex mu;
  static std::unordered_map<const void*, int> limit;
  std::lock_guard<std::mutex> lock(mu);
  auto it = limit.find(kernel);
  if (it != limit.end() && it->second >= bytes) return MINITP_OK;
  MINITP_RETURN_HIP(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
  limit[kernel] = bytes;
  return MINITP_OK;
}

}  // namespace minitp
