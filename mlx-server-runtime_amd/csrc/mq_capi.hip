// C ABI of libmi355q: argument validation, then dispatch to the kernels.
// Declarations and the reference interface each entry point replaces are in
// include/mq.h.
#include <cstdarg>
#include <cstdio>

#include "../../include/mq.h"
#include "mq_internal.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return MQ_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(MQ_ERR_HIP, "[%s] HIP launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

}  // namespace

int mq::set_last_error(int code, const char* msg) {
  snprintf(g_err, sizeof(g_err), "%s", msg);
  return code;
}

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int64_t kMaxDim = (int64_t)1 << 31;

// GEMV kernel for decode-sized M.  Measured on MI355X: the dot2 kernel streams
// large matrices faster at M <= 2 (its 256-byte row segments per load beat the
// matrix-core kernel's 64-byte ones), the matrix-core kernel wins everywhere
// else (its VALU cost does not grow with M).
bool use_matrix_core_gemv(int64_t M, int64_t N, int64_t K) {
  return !(M <= 2 && N * K >= ((int64_t)1 << 25));
}

// Checks shared by every entry point, in the order MLX reports them.
int check_quant(const char* op, int64_t K, int group_size, int bits) {
  if (bits != 2 && bits != 3 && bits != 4 && bits != 5 && bits != 6 && bits != 8)
    return fail(MQ_ERR_INVALID,
                "[%s] The requested number of bits %d is not supported. The supported bits are "
                "2, 3, 4, 5, 6 and 8.",
                op, bits);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(MQ_ERR_INVALID,
                "[%s] The requested group size %d is not supported. The supported group sizes "
                "are 32, 64 and 128.",
                op, group_size);
  if (K <= 0 || K % group_size != 0)
    return fail(MQ_ERR_INVALID,
                "[%s] The last dimension of the matrix needs to be divisible by the "
                "quantization group size %d. However the provided matrix has %lld columns.",
                op, group_size, (long long)K);
  if (K >= kMaxDim) return fail(MQ_ERR_INVALID, "[%s] K=%lld is too large.", op, (long long)K);
  return MQ_OK;
}

// 2, 3, 5 and 6 bits (codes as one bit stream per row): quantize, dequantize,
// the embedding lookup and mq_quantized_matmul_ws (through its workspace) take
// them; the other matmul entry points run word-aligned codes only.
bool stream_bits(int bits) { return bits != 4 && bits != 8; }

int check_word_bits(const char* op, int bits) {
  if (stream_bits(bits))
    return fail(MQ_ERR_UNSUPPORTED,
                "[%s] bits=%d codes run here as one byte each: repack them with "
                "mq_repack_codes_u8 and call with bits=8 (or use mq_quantized_matmul_ws).",
                op, bits);
  return MQ_OK;
}

// Repacked 8-bit codes of an N x K matrix, at the start of the workspace.
size_t repack_bytes(int64_t N, int64_t K) { return (size_t)((N * K + 255) / 256 * 256); }

int check_dim(const char* op, const char* name, int64_t v) {
  if (v < 0 || v >= kMaxDim)
    return fail(MQ_ERR_INVALID, "[%s] %s=%lld is out of range.", op, name, (long long)v);
  return MQ_OK;
}

// The matrix-core GEMV for a dense matmul. It takes 8-bit rows up to 16,
// but at 9..16 rows the skinny GEMM's one 32-row tile streams the codes
// faster (M = 16, K = 3584: N = 18944 29.4 us against 34.6, N = 4608
// 11.4 us against 14.1), so there it only serves shapes the skinny GEMM
// does not fit.
// The matrix-core GEMV reads one scale per 64-wide k step (group size 64); the
// other kernels take group sizes 32, 64 and 128.
bool dense_gemv(int64_t M, int64_t N, int64_t K, int bits, int group_size) {
  return group_size == 64 && mq::qmvm_fits(M, N, K, bits, 1) &&
         (M <= 8 || !mq::qmms_fits(M, N, K, bits));
}

// The kernel mq_quantized_matmul_ws runs for 4- or 8-bit codes (group size
// 32, 64 or 128 dividing K), in its order of preference.
enum class Dense { kNone, kQmv1, kQmvm, kQmv, kSkinny, kQmm4, kQmm };

Dense dense_path(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  if (mq::qmv1_plain_fits(M, N, K, bits, group_size)) return Dense::kQmv1;
  const bool qmv = mq::qmv_fits(M, N, K, bits, 1, group_size);
  if (dense_gemv(M, N, K, bits, group_size) && (use_matrix_core_gemv(M, N, K) || !qmv))
    return Dense::kQmvm;
  if (qmv) return Dense::kQmv;
  // the skinny MFMA kernel above the GEMV range, up to two 128-row tiles
  if (M <= 256 && !dense_gemv(M, N, K, bits, group_size) && mq::qmms_fits(M, N, K, bits))
    return Dense::kSkinny;
  if (mq::qmm4_fits(M, N, K, bits, group_size)) return Dense::kQmm4;
  // Taller shapes with too few 256 x 256 tiles for the large-M GEMM: the
  // skinny GEMM's 64- or 128-row tiles and K splits fill the GPU where the
  // 128 x 128 tiles of the plain GEMM do not (M x N x K = 4096 x 128 x 2048,
  // a MoE router at prefill: 35.1 -> 14.8 us a call; 2048 x 256 x 2048 35.1
  // -> 14.5; 1024 x 1024 x 1024 20.1 -> 15.7).  Its partial sums take at
  // most 256 tiles of 128 x 128 floats (16 MiB).
  if (mq::qmms_fits(M, N, K, bits)) return Dense::kSkinny;
  return K % 64 ? Dense::kNone : Dense::kQmm;
}

// bits 4 or 8 and a group size that divides K (the matmul entries' checks)
bool word_shape(int64_t K, int group_size, int bits) {
  return (bits == 4 || bits == 8) && (group_size == 32 || group_size == 64 || group_size == 128) &&
         K % group_size == 0;
}

}  // namespace

extern "C" {

int mq_version(void) { return (2 << 16) | 2; }

const char* mq_last_error(void) { return g_err; }

int mq_quantize(const mq_bf16* w, uint32_t* wq, mq_bf16* scales, mq_bf16* biases, int64_t rows,
                int64_t K, int group_size, int bits, hipStream_t stream) {
  const char* op = "quantize";
  if (int rc = check_quant(op, K, group_size, bits)) return rc;
  if (int rc = check_dim(op, "rows", rows)) return rc;
  if (rows == 0) return ok();
  if (!w || !wq || !scales || !biases) return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(w) || !aligned16(wq))
    return fail(MQ_ERR_INVALID, "[%s] w and wq must be 16-byte aligned.", op);
  return hip_status(mq::launch_quantize(w, wq, scales, biases, rows, K, group_size, bits, stream),
                    op);
}

int mq_dequantize(const uint32_t* wq, const mq_bf16* scales, const mq_bf16* biases, mq_bf16* out,
                  int64_t rows, int64_t K, int group_size, int bits, hipStream_t stream) {
  const char* op = "dequantize";
  if (int rc = check_quant(op, K, group_size, bits)) return rc;
  if (int rc = check_dim(op, "rows", rows)) return rc;
  if (rows == 0) return ok();
  if (!wq || !scales || !biases || !out) return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(wq) || !aligned16(out))
    return fail(MQ_ERR_INVALID, "[%s] wq and out must be 16-byte aligned.", op);
  return hip_status(
      mq::launch_dequantize(wq, scales, biases, nullptr, rows, rows, out, K, group_size, bits,
                            stream),
      op);
}

int mq_embedding_lookup(const int32_t* ids, int64_t n_ids, const uint32_t* wq,
                        const mq_bf16* scales, const mq_bf16* biases, int64_t rows, int64_t K,
                        int group_size, int bits, mq_bf16* out, hipStream_t stream) {
  const char* op = "embedding_lookup";
  if (int rc = check_quant(op, K, group_size, bits)) return rc;
  if (int rc = check_dim(op, "rows", rows)) return rc;
  if (int rc = check_dim(op, "n_ids", n_ids)) return rc;
  if (n_ids == 0) return ok();
  if (!ids || !wq || !scales || !biases || !out)
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(wq) || !aligned16(out))
    return fail(MQ_ERR_INVALID, "[%s] wq and out must be 16-byte aligned.", op);
  return hip_status(
      mq::launch_dequantize(wq, scales, biases, ids, n_ids, rows, out, K, group_size, bits,
                            stream),
      op);
}

int mq_repack_codes_u8(const uint32_t* wq, uint32_t* wq8, int64_t rows, int64_t K, int bits,
                       hipStream_t stream) {
  const char* op = "repack_codes_u8";
  if (bits != 2 && bits != 3 && bits != 5 && bits != 6)
    return fail(MQ_ERR_INVALID, "[%s] bits=%d: only 2, 3, 5 and 6-bit codes are repacked.", op,
                bits);
  if (K <= 0 || K % 32 || K >= kMaxDim)
    return fail(MQ_ERR_INVALID, "[%s] K=%lld must be a positive multiple of 32.", op,
                (long long)K);
  if (int rc = check_dim(op, "rows", rows)) return rc;
  if (rows == 0) return ok();
  if (!wq || !wq8) return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(wq8)) return fail(MQ_ERR_INVALID, "[%s] wq8 must be 16-byte aligned.", op);
  return hip_status(mq::launch_repack_u8(wq, wq8, rows, K, bits, stream), op);
}

size_t mq_quantized_matmul_workspace(int64_t M, int64_t N, int64_t K, int group_size,
                                     int bits) {
  if (M <= 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim) return 0;
  if ((bits == 2 || bits == 3 || bits == 5 || bits == 6) &&
      (group_size == 32 || group_size == 64 || group_size == 128) && K % group_size == 0) {
    if (mq::qmvs_fits(M, N, K, bits, group_size)) return 0;  // read at their width
    return repack_bytes(N, K) + mq_quantized_matmul_workspace(M, N, K, group_size, 8);
  }
  if (!word_shape(K, group_size, bits)) return 0;
  switch (dense_path(M, N, K, group_size, bits)) {
    case Dense::kSkinny: return mq::qmms_workspace_bytes(M, N, K, bits);
    case Dense::kQmm4: return mq::qmm4_workspace_bytes(M, N, K, group_size);
    default: return 0;
  }
}

}  // extern "C"

namespace mq {
// Whether mq_quantized_matmul_ws runs a shape with less workspace than
// mq_quantized_matmul_workspace asks for: the large-M GEMM's stream-K plan,
// which without its workspace runs every tile whole.
bool qmm_workspace_optional(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  if (M <= 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim) return false;
  if (!word_shape(K, group_size, bits)) return false;
  return dense_path(M, N, K, group_size, bits) == Dense::kQmm4 &&
         mq::qmm4_stream_k(M, N, K, group_size);
}
}  // namespace mq

namespace {
// How mq_quantized_matmul_swiglu runs a shape: 1 the dot2 GEMV with the SwiGLU
// epilogue (where mq_quantized_matmul itself runs that GEMV on the 2N rows),
// 2 the skinny GEMM's K splits with a SwiGLU reduce (where mq_quantized_matmul
// with its workspace splits K), 3 the unsplit one-tile skinny GEMM with the
// SwiGLU in its epilogue, 4 the large-M GEMM with the SwiGLU in its epilogue
// (where mq_quantized_matmul runs that GEMM unsplit), 0 not fused.
int swiglu_route(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  if (M <= 0 || N <= 0 || K <= 0 || M >= kMaxDim || 2 * N >= kMaxDim || K >= kMaxDim) return 0;
  if (!word_shape(K, group_size, bits)) return 0;
  // what mq_quantized_matmul runs on the 2N rows
  const int64_t N2 = 2 * N;
  switch (dense_path(M, N2, K, group_size, bits)) {
    case Dense::kQmv1: return mq::qmv1_fits(M, N2, K, bits, group_size) ? 1 : 0;
    case Dense::kQmv: return mq::qmv_swiglu_fits(M, N, K, bits, group_size) ? 1 : 0;
    case Dense::kSkinny:
      if (mq::qmms_split_fusable(M, N2, K, bits)) return 2;
      return mq::qmms_swiglu_direct(M, N, K, bits) ? 3 : 0;
    case Dense::kQmm4:
      // only with no even K split: the fused kernel runs every tile whole, as
      // mq_quantized_matmul_ws does without a workspace (the same kernel, so
      // the same bits; with one, a stream-K plan may sum a short last round
      // of tiles in pieces)
      return mq::qmm4_unsplit(M, N2, K, group_size) &&
                     mq::qmm4_swiglu_fits(M, N, K, bits, group_size)
                 ? 4
                 : 0;
    default: return 0;
  }
}

// mq_quantized_matmul_add_rms_norm takes the skinny GEMM's split plans (the
// reduce ends in the norm) for rows of at most 8192.
bool add_norm_fusable(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  if (M <= 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim) return false;
  if (!word_shape(K, group_size, bits) || N % 8 || N > 8192) return false;
  return dense_path(M, N, K, group_size, bits) == Dense::kSkinny &&
         mq::qmms_split_fusable(M, N, K, bits);
}
}  // namespace

extern "C" {

int mq_quantized_matmul_swiglu_supported(int64_t M, int64_t N, int64_t K, int group_size,
                                         int bits) {
  return swiglu_route(M, N, K, group_size, bits) != 0 ? 1 : 0;
}

size_t mq_quantized_matmul_swiglu_workspace(int64_t M, int64_t N, int64_t K, int group_size,
                                            int bits) {
  if (swiglu_route(M, N, K, group_size, bits) != 2) return 0;
  return mq::qmms_workspace_bytes(M, 2 * N, K, bits);
}

int mq_quantized_matmul_swiglu_ws(const mq_bf16* x, const uint32_t* wq, const mq_bf16* scales,
                                  const mq_bf16* biases, mq_bf16* y, int64_t M, int64_t N,
                                  int64_t K, int group_size, int bits, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
  const char* op = "quantized_matmul_swiglu";
  if (int rc = check_quant(op, K, group_size, bits)) return rc;
  if (int rc = check_word_bits(op, bits)) return rc;
  if (int rc = check_dim(op, "M", M)) return rc;
  if (int rc = check_dim(op, "N", 2 * N)) return rc;
  if (M == 0 || N == 0) return ok();
  const int route = swiglu_route(M, N, K, group_size, bits);
  if (!route)
    return fail(MQ_ERR_UNSUPPORTED,
                "[%s] M=%lld, N=%lld, K=%lld is not a fused shape; use mq_quantized_matmul and "
                "mq_silu_mul.",
                op, (long long)M, (long long)N, (long long)K);
  if (!x || !wq || !scales || !biases || !y) return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(x) || !aligned16(wq))
    return fail(MQ_ERR_INVALID, "[%s] x and wq must be 16-byte aligned.", op);
  if (route == 1)
    return hip_status(
        mq::launch_qmv_swiglu(x, wq, scales, biases, y, M, N, K, bits, group_size, stream), op);
  if (route == 3)
    return hip_status(
        mq::launch_qmms_swiglu_direct(x, wq, scales, biases, y, M, N, K, bits, group_size,
                                      stream),
        op);
  if (route == 4)
    return hip_status(
        mq::launch_qmm4_swiglu(x, wq, scales, biases, y, M, N, K, bits, group_size, stream),
                      op);
  const size_t need = mq::qmms_workspace_bytes(M, 2 * N, K, bits);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(MQ_ERR_INVALID,
                "[%s] this shape needs a 16-byte aligned workspace of %zu bytes "
                "(mq_quantized_matmul_swiglu_workspace).",
                op, need);
  return hip_status(mq::launch_qmms_swiglu(x, wq, scales, biases, y, M, N, K, bits, group_size,
                                           workspace, workspace_bytes, stream),
                    op);
}

int mq_quantized_matmul_swiglu(const mq_bf16* x, const uint32_t* wq, const mq_bf16* scales,
                               const mq_bf16* biases, mq_bf16* y, int64_t M, int64_t N, int64_t K,
                               int group_size, int bits, hipStream_t stream) {
  return mq_quantized_matmul_swiglu_ws(x, wq, scales, biases, y, M, N, K, group_size, bits,
                                       nullptr, 0, stream);
}

int mq_quantized_matmul_add_rms_norm_supported(int64_t M, int64_t N, int64_t K, int group_size,
                                               int bits) {
  return add_norm_fusable(M, N, K, group_size, bits) ? 1 : 0;
}

size_t mq_quantized_matmul_add_rms_norm_workspace(int64_t M, int64_t N, int64_t K,
                                                  int group_size, int bits) {
  return add_norm_fusable(M, N, K, group_size, bits) ? mq::qmms_workspace_bytes(M, N, K, bits)
                                                     : 0;
}

int mq_quantized_matmul_add_rms_norm(const mq_bf16* x, const uint32_t* wq, const mq_bf16* scales,
                                     const mq_bf16* biases, const mq_bf16* bias_vec,
                                     const mq_bf16* residual, mq_bf16* residual_out,
                                     const mq_bf16* norm_weight, float eps, mq_bf16* out,
                                     int64_t M, int64_t N, int64_t K, int group_size, int bits,
                                     void* workspace, size_t workspace_bytes,
                                     hipStream_t stream) {
  const char* op = "quantized_matmul_add_rms_norm";
  if (int rc = check_quant(op, K, group_size, bits)) return rc;
  if (int rc = check_word_bits(op, bits)) return rc;
  if (int rc = check_dim(op, "M", M)) return rc;
  if (int rc = check_dim(op, "N", N)) return rc;
  if (M == 0 || N == 0) return ok();
  if (!add_norm_fusable(M, N, K, group_size, bits))
    return fail(MQ_ERR_UNSUPPORTED,
                "[%s] M=%lld, N=%lld, K=%lld is not a fused shape (a split skinny GEMM, N <= "
                "8192); use mq_quantized_matmul_ws and mq_rms_norm.",
                op, (long long)M, (long long)N, (long long)K);
  if (!x || !wq || !scales || !biases || !residual || !residual_out || !norm_weight || !out)
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(x) || !aligned16(wq) || !aligned16(residual) || !aligned16(residual_out) ||
      !aligned16(norm_weight) || !aligned16(out))
    return fail(MQ_ERR_INVALID, "[%s] x, wq, residual, residual_out, norm_weight and out must be "
                "16-byte aligned.", op);
  const size_t need = mq::qmms_workspace_bytes(M, N, K, bits);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(MQ_ERR_INVALID,
                "[%s] this shape needs a 16-byte aligned workspace of %zu bytes "
                "(mq_quantized_matmul_add_rms_norm_workspace).",
                op, need);
  return hip_status(mq::launch_qmms_add_norm(x, wq, scales, biases, bias_vec, residual,
                                             residual_out, norm_weight, eps, out, M, N, K, bits,
                                             group_size, workspace, workspace_bytes, stream),
                    op);
}

int mq_rms_norm_quantized_matmul_supported(int64_t M, int64_t N, int64_t K, int group_size,
                                           int bits, int swiglu) {
  if (M != 1 || N <= 0 || K <= 0 || 2 * N >= kMaxDim || K >= kMaxDim) return 0;
  if (mq::qmv1_fits(1, swiglu ? 2 * N : N, K, bits, group_size)) return 1;
  if (!word_shape(K, group_size, bits)) return 0;
  return mq::qmv_norm_fits(N, K, bits, swiglu != 0, group_size) ? 1 : 0;
}

namespace {
bool overlap(const void* a, const void* b, int64_t bytes) {
  const char *pa = static_cast<const char*>(a), *pb = static_cast<const char*>(b);
  return pa < pb + bytes && pb < pa + bytes;
}
}  // namespace

int mq_rms_norm_quantized_matmul(const mq_bf16* a, const mq_bf16* residual, mq_bf16* residual_out,
                                 const mq_bf16* norm_weight, float eps, const uint32_t* wq,
                                 const mq_bf16* scales, const mq_bf16* biases,
                                 const mq_bf16* bias_vec, mq_bf16* y, int64_t M, int64_t N,
                                 int64_t K, int group_size, int bits, int swiglu,
                                 hipStream_t stream) {
  const char* op = "rms_norm_quantized_matmul";
  if (int rc = check_quant(op, K, group_size, bits)) return rc;
  if (int rc = check_word_bits(op, bits)) return rc;
  if (int rc = check_dim(op, "M", M)) return rc;
  if (int rc = check_dim(op, "N", swiglu ? 2 * N : N)) return rc;
  if (M == 0 || N == 0) return ok();
  if (!mq_rms_norm_quantized_matmul_supported(M, N, K, group_size, bits, swiglu))
    return fail(MQ_ERR_UNSUPPORTED,
                "[%s] M=%lld, N=%lld, K=%lld%s is not a fused shape (one row, K <= 8192); use "
                "mq_rms_norm and mq_quantized_matmul.",
                op, (long long)M, (long long)N, (long long)K, swiglu ? " (SwiGLU)" : "");
  if (swiglu && bias_vec)
    return fail(MQ_ERR_INVALID, "[%s] the SwiGLU form takes no bias.", op);
  if (!residual != !residual_out)
    return fail(MQ_ERR_INVALID, "[%s] residual and residual_out go together.", op);
  if (!a || !norm_weight || !wq || !scales || !biases || !y)
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(a) || !aligned16(norm_weight) || !aligned16(wq) ||
      (residual && (!aligned16(residual) || !aligned16(residual_out))))
    return fail(MQ_ERR_INVALID, "[%s] a, residual, residual_out, norm_weight and wq must be "
                "16-byte aligned.", op);
  // Every block reads a and residual while the first one writes residual_out.
  if (residual_out && (overlap(residual_out, residual, K * 2) || overlap(residual_out, a, K * 2)))
    return fail(MQ_ERR_INVALID, "[%s] residual_out may not overlap a or residual.", op);
  return hip_status(mq::launch_qmv_norm(a, residual, residual_out, norm_weight, eps, wq, scales,
                                        biases, bias_vec, y, N, K, bits, swiglu != 0, group_size,
                                        stream),
                    op);
}

int mq_quantized_matmul(const mq_bf16* x, const uint32_t* wq, const mq_bf16* scales,
                        const mq_bf16* biases, const mq_bf16* bias_vec, mq_bf16* y, int64_t M,
                        int64_t N, int64_t K, int group_size, int bits, int transpose,
                        hipStream_t stream) {
  return mq_quantized_matmul_ws(x, wq, scales, biases, bias_vec, y, M, N, K, group_size, bits,
                                transpose, nullptr, 0, stream);
}

int mq_quantized_matmul_ws(const mq_bf16* x, const uint32_t* wq, const mq_bf16* scales,
                           const mq_bf16* biases, const mq_bf16* bias_vec, mq_bf16* y, int64_t M,
                           int64_t N, int64_t K, int group_size, int bits, int transpose,
                           void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const char* op = "quantized_matmul";
  if (int rc = check_quant(op, K, group_size, bits)) return rc;
  if (int rc = check_dim(op, "M", M)) return rc;
  if (int rc = check_dim(op, "N", N)) return rc;
  if (!transpose)
    return fail(MQ_ERR_UNSUPPORTED, "[%s] transpose=False is not implemented on this backend.",
                op);
  if (M == 0 || N == 0) return ok();
  if (!x || !wq || !scales || !biases || !y) return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(x) || !aligned16(wq))
    return fail(MQ_ERR_INVALID, "[%s] x and wq must be 16-byte aligned.", op);
  if ((M + 127) / 128 > 65535)
    return fail(MQ_ERR_UNSUPPORTED, "[%s] M=%lld exceeds the launch grid (8388480 rows).", op,
                (long long)M);
  if (stream_bits(bits) && mq::qmvs_fits(M, N, K, bits, group_size))
    return hip_status(mq::launch_qmvs(x, wq, scales, biases, bias_vec, y, N, K, bits,
                                      group_size, stream),
                      op);
  if (stream_bits(bits)) {
    // codes rewritten one byte each into the workspace, then the 8-bit
    // kernels with the rest of it (same scales and biases: the dequantized
    // weights are those of the bits-wide codes)
    const size_t rb = repack_bytes(N, K);
    // the one refusal of the 8-bit path below, checked before the repack so
    // that a failed call enqueues nothing
    if (dense_path(M, N, K, group_size, 8) == Dense::kNone)
      return fail(MQ_ERR_UNSUPPORTED,
                  "[%s] M=%lld rows with K=%lld (not a multiple of 64) are not implemented on "
                  "this backend.",
                  op, (long long)M, (long long)K);
    if (!workspace || workspace_bytes < rb || !aligned16(workspace))
      return fail(MQ_ERR_UNSUPPORTED,
                  "[%s] bits=%d needs a 16-byte aligned workspace of at least %zu bytes for its "
                  "codes repacked to 8 bits (mq_quantized_matmul_workspace).",
                  op, bits, rb);
    uint32_t* wq8 = static_cast<uint32_t*>(workspace);
    if (hipError_t e = mq::launch_repack_u8(wq, wq8, N, K, bits, stream); e != hipSuccess)
      return hip_status(e, op);
    return mq_quantized_matmul_ws(x, wq8, scales, biases, bias_vec, y, M, N, K, group_size, 8, 1,
                                  static_cast<char*>(workspace) + rb, workspace_bytes - rb,
                                  stream);
  }
  hipError_t e;
  const mq::GatherMap g1{nullptr, nullptr, 1, 1, 1};
  const Dense path = dense_path(M, N, K, group_size, bits);
  if ((path == Dense::kSkinny || path == Dense::kQmm4) && workspace && !aligned16(workspace))
    return fail(MQ_ERR_INVALID, "[%s] the workspace must be 16-byte aligned.", op);
  switch (path) {
    case Dense::kQmv1:
      e = mq::launch_qmv1(x, wq, scales, biases, bias_vec, y, N, K, group_size, false, nullptr,
                          stream);
      break;
    case Dense::kQmvm:
      e = mq::launch_qmvm(x, wq, scales, biases, bias_vec, y, M, N, K, bits, g1, stream);
      break;
    case Dense::kQmv:
      e = mq::launch_qmv(x, wq, scales, biases, bias_vec, y, M, N, K, bits, g1, group_size,
                         stream);
      break;
    case Dense::kSkinny:
      e = mq::launch_qmms(x, wq, scales, biases, bias_vec, y, M, N, K, bits, group_size,
                          workspace, workspace_bytes, stream);
      break;
    case Dense::kQmm4:
      e = mq::launch_qmm4(x, wq, scales, biases, bias_vec, y, M, N, K, bits, group_size,
                          workspace, workspace_bytes, stream);
      break;
    case Dense::kQmm:
      e = mq::launch_qmm(x, wq, scales, biases, bias_vec, y, M, N, K, group_size, bits, stream);
      break;
    default:
      return fail(MQ_ERR_UNSUPPORTED,
                  "[%s] M=%lld rows with K=%lld (not a multiple of 64) are not implemented on "
                  "this backend.",
                  op, (long long)M, (long long)K);
  }
  return hip_status(e, op);
}

int mq_gather_qmm(const mq_bf16* x, const int32_t* lhs_indices, const int32_t* rhs_indices,
                  const uint32_t* wq, const mq_bf16* scales, const mq_bf16* biases, mq_bf16* y,
                  int64_t T, int64_t M, int64_t N, int64_t K, int64_t E, int64_t x_batches,
                  int group_size, int bits, int transpose, int sorted_indices,
                  hipStream_t stream) {
  const char* op = "gather_qmm";
  if (int rc = check_quant(op, K, group_size, bits)) return rc;
  if (int rc = check_word_bits(op, bits)) return rc;
  if (int rc = check_dim(op, "T", T)) return rc;
  if (int rc = check_dim(op, "M", M)) return rc;
  if (int rc = check_dim(op, "N", N)) return rc;
  if (int rc = check_dim(op, "E", E)) return rc;
  if (int rc = check_dim(op, "x_batches", x_batches)) return rc;
  if (!transpose)
    return fail(MQ_ERR_UNSUPPORTED, "[%s] transpose=False is not implemented on this backend.",
                op);
  if (T * M >= kMaxDim) return fail(MQ_ERR_INVALID, "[%s] T*M is too large.", op);
  if (!lhs_indices && x_batches != T)
    return fail(MQ_ERR_INVALID, "[%s] without lhs_indices x must have T=%lld batches, got %lld.",
                op, (long long)T, (long long)x_batches);
  if (T == 0 || M == 0 || N == 0) return ok();
  if (E == 0) return fail(MQ_ERR_INVALID, "[%s] the expert table is empty.", op);
  if (!x || !rhs_indices || !wq || !scales || !biases || !y)
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(x) || !aligned16(wq))
    return fail(MQ_ERR_INVALID, "[%s] x and wq must be 16-byte aligned.", op);
  if ((T * M + 127) / 128 > 65535)
    return fail(MQ_ERR_UNSUPPORTED, "[%s] T*M=%lld exceeds the launch grid (8388480 rows).", op,
                (long long)(T * M));
  hipError_t e;
  // Few rows: one GEMV block row per (t, N tile); each t streams its expert.
  // Many rows: MFMA tiles over the (expert-sorted) rows.
  const mq::GatherMap g{lhs_indices, rhs_indices, T, E, x_batches};
  const bool few = T * M <= 64 || !sorted_indices;
  // Single-row batches (a decode step's (token, expert) pairs) are many small
  // GEMVs: the dot2 kernel streams them faster than the matrix-core one
  // (measured on the 128-expert, 2048 x 768 banks at 64 pairs: 25 % faster
  // decode).
  const bool dot2_rows = M <= 2 && T > 1;
  if (few && group_size == 64 && mq::qmvm_fits(M, N, K, bits, T) &&
      ((use_matrix_core_gemv(M, N, K) && !dot2_rows) || !mq::qmv_fits(M, N, K, bits, T, 64))) {
    e = mq::launch_qmvm(x, wq, scales, biases, nullptr, y, M, N, K, bits, g, stream);
  } else if (few && mq::qmv_fits(M, N, K, bits, T, group_size)) {
    e = mq::launch_qmv(x, wq, scales, biases, nullptr, y, M, N, K, bits, g, group_size,
                       stream);
  } else if (sorted_indices && mq::qmm4_gather_fits(T, M, N, K, E, x_batches, bits, group_size)) {
    e = mq::launch_qmm4_gather(x, lhs_indices, rhs_indices, nullptr, wq, scales, biases, y, T, M,
                               N, K, E, x_batches, bits, group_size, false, stream);
  } else {
    if (K % 64)
      return fail(MQ_ERR_UNSUPPORTED,
                  "[%s] T*M=%lld rows with K=%lld (not a multiple of 64) are not implemented on "
                  "this backend.",
                  op, (long long)(T * M), (long long)K);
    e = mq::launch_gather_qmm_rows(x, lhs_indices, rhs_indices, wq, scales, biases, y, T * M, N,
                                   K, E, x_batches * M, (int)M, group_size, bits, stream);
  }
  return hip_status(e, op);
}

int mq_gather_qmm_segments(const mq_bf16* x, const int32_t* lhs_indices,
                           const int32_t* rhs_indices, const int32_t* expert_offsets,
                           const uint32_t* wq, const mq_bf16* scales, const mq_bf16* biases,
                           mq_bf16* y, int64_t T, int64_t M, int64_t N, int64_t K, int64_t E,
                           int64_t x_batches, int group_size, int bits, int swiglu,
                           hipStream_t stream) {
  const char* op = swiglu ? "gather_qmm_swiglu" : "gather_qmm";
  if (!expert_offsets) return fail(MQ_ERR_INVALID, "[%s] expert_offsets is null.", op);
  if (int rc = check_quant(op, K, group_size, bits)) return rc;
  if (int rc = check_word_bits(op, bits)) return rc;
  if (int rc = check_dim(op, "T", T)) return rc;
  if (int rc = check_dim(op, "M", M)) return rc;
  if (int rc = check_dim(op, "N", swiglu ? 2 * N : N)) return rc;
  if (int rc = check_dim(op, "E", E)) return rc;
  if (int rc = check_dim(op, "x_batches", x_batches)) return rc;
  if (T * M >= kMaxDim) return fail(MQ_ERR_INVALID, "[%s] T*M is too large.", op);
  if (!lhs_indices && x_batches != T)
    return fail(MQ_ERR_INVALID, "[%s] without lhs_indices x must have T=%lld batches, got %lld.",
                op, (long long)T, (long long)x_batches);
  if (T == 0 || M == 0 || N == 0) return ok();
  if (E == 0) return fail(MQ_ERR_INVALID, "[%s] the expert table is empty.", op);
  if (!x || !rhs_indices || !wq || !scales || !biases || !y)
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(x) || !aligned16(wq))
    return fail(MQ_ERR_INVALID, "[%s] x and wq must be 16-byte aligned.", op);
  // Decode-sized batches run as mq_gather_qmm (or its SwiGLU GEMV) does: the
  // offsets are not needed there.
  const bool fits =
      mq::qmm4_gather_fits(T, M, swiglu ? 2 * N : N, K, E, x_batches, bits, group_size);
  if (T * M <= 64 || !fits) {
    if (!swiglu)
      return mq_gather_qmm(x, lhs_indices, rhs_indices, wq, scales, biases, y, T, M, N, K, E,
                           x_batches, group_size, bits, 1, 1, stream);
    if (mq_gather_qmm_swiglu_supported(T, M, N, K, group_size, bits))
      return mq_gather_qmm_swiglu(x, lhs_indices, rhs_indices, wq, scales, biases, y, T, M, N,
                                  K, E, x_batches, group_size, bits, stream);
    return fail(MQ_ERR_UNSUPPORTED,
                "[%s] T=%lld, M=%lld, N=%lld, K=%lld is not a fused shape; use "
                "mq_gather_qmm_segments and mq_silu_mul.",
                op, (long long)T, (long long)M, (long long)N, (long long)K);
  }
  return hip_status(mq::launch_qmm4_gather(x, lhs_indices, rhs_indices, expert_offsets, wq,
                                           scales, biases, y, T, M, N, K, E, x_batches, bits,
                                           group_size, swiglu != 0, stream),
                    op);
}

int mq_gather_qmm_segments_supported(int64_t T, int64_t M, int64_t N, int64_t K, int64_t E,
                                     int64_t x_batches, int group_size, int bits, int swiglu) {
  if (bits != 2 && bits != 3 && bits != 4 && bits != 5 && bits != 6 && bits != 8) return 0;
  if (group_size != 32 && group_size != 64 && group_size != 128) return 0;
  if (T < 0 || M < 0 || N < 0 || K < 1 || E < 1 || x_batches < 0 || K % group_size) return 0;
  if (T >= kMaxDim || M >= kMaxDim || 2 * N >= kMaxDim || K >= kMaxDim || E >= kMaxDim ||
      x_batches >= kMaxDim || T * M >= kMaxDim)
    return 0;
  if (!swiglu) return bits == 4 || bits == 8;
  if (bits != 4 && bits != 8) return 0;
  if (T * M > 64 && mq::qmm4_gather_fits(T, M, 2 * N, K, E, x_batches, bits, group_size))
    return 1;
  return mq_gather_qmm_swiglu_supported(T, M, N, K, group_size, bits);
}

int mq_gather_qmm_swiglu_supported(int64_t T, int64_t M, int64_t N, int64_t K, int group_size,
                                   int bits) {
  if (K < 1 || !word_shape(K, group_size, bits)) return 0;
  // Only where mq_gather_qmm itself runs the per-pair GEMV (at most 64 rows in
  // all): more pairs go to the sorted gather GEMM, which reads each expert once.
  if (T * M > 64) return 0;
  return mq::gather_qmv_swiglu_fits(M, N, K, bits, T, group_size) ? 1 : 0;
}

int mq_gather_qmm_swiglu(const mq_bf16* x, const int32_t* lhs_indices,
                         const int32_t* rhs_indices, const uint32_t* wq, const mq_bf16* scales,
                         const mq_bf16* biases, mq_bf16* y, int64_t T, int64_t M, int64_t N,
                         int64_t K, int64_t E, int64_t x_batches, int group_size, int bits,
                         hipStream_t stream) {
  const char* op = "gather_qmm_swiglu";
  if (int rc = check_quant(op, K, group_size, bits)) return rc;
  if (int rc = check_word_bits(op, bits)) return rc;
  if (int rc = check_dim(op, "T", T)) return rc;
  if (int rc = check_dim(op, "M", M)) return rc;
  if (int rc = check_dim(op, "N", N)) return rc;
  if (int rc = check_dim(op, "E", E)) return rc;
  if (int rc = check_dim(op, "x_batches", x_batches)) return rc;
  if (!lhs_indices && x_batches != T)
    return fail(MQ_ERR_INVALID, "[%s] without lhs_indices x must have T=%lld batches, got %lld.",
                op, (long long)T, (long long)x_batches);
  if (T == 0 || M == 0 || N == 0) return ok();
  if (!mq_gather_qmm_swiglu_supported(T, M, N, K, group_size, bits))
    return fail(MQ_ERR_UNSUPPORTED,
                "[%s] T=%lld M=%lld N=%lld K=%lld is not a shape the fused kernel takes "
                "(mq_gather_qmm_swiglu_supported).",
                op, (long long)T, (long long)M, (long long)N, (long long)K);
  if (E == 0) return fail(MQ_ERR_INVALID, "[%s] the expert table is empty.", op);
  if (!x || !rhs_indices || !wq || !scales || !biases || !y)
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(x) || !aligned16(wq))
    return fail(MQ_ERR_INVALID, "[%s] x and wq must be 16-byte aligned.", op);
  const mq::GatherMap g{lhs_indices, rhs_indices, T, E, x_batches};
  return hip_status(
      mq::launch_gather_qmv_swiglu(x, wq, scales, biases, y, M, N, K, bits, g, group_size,
                                   stream),
      op);
}

int mq_rms_norm(const mq_bf16* x, const mq_bf16* residual, mq_bf16* residual_out,
                const mq_bf16* weight, mq_bf16* out, int64_t rows, int64_t dim, float eps,
                hipStream_t stream) {
  const char* op = "rms_norm";
  if (int rc = check_dim(op, "rows", rows)) return rc;
  if (!mq::rmsnorm_supported(dim))
    return fail(MQ_ERR_UNSUPPORTED, "[%s] dim=%lld is not supported (a multiple of 8, <= 8192).",
                op, (long long)dim);
  if (!residual != !residual_out)
    return fail(MQ_ERR_INVALID, "[%s] residual and residual_out go together.", op);
  if (rows == 0) return ok();
  if (!x || !weight || !out) return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out) ||
      (residual && (!aligned16(residual) || !aligned16(residual_out))))
    return fail(MQ_ERR_INVALID, "[%s] every buffer must be 16-byte aligned.", op);
  return hip_status(
      mq::launch_rmsnorm(x, residual, residual_out, weight, out, rows, dim, eps, stream), op);
}

namespace {
int check_pages(const char* op, int64_t B, int n_heads, int n_kv_heads, int64_t pages_per_seq,
                int64_t page_size, int64_t num_pages) {
  if (int rc = check_dim(op, "batch", B)) return rc;
  if (B > 65535) return fail(MQ_ERR_UNSUPPORTED, "[%s] batch=%lld > 65535.", op, (long long)B);
  if (n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads)
    return fail(MQ_ERR_INVALID, "[%s] query heads must be divisible by KV heads (%d, %d).", op,
                n_heads, n_kv_heads);
  if (page_size <= 0 || pages_per_seq <= 0 || num_pages <= 0)
    return fail(MQ_ERR_INVALID, "[%s] page_size, pages_per_seq and num_pages must be > 0.", op);
  if (pages_per_seq * page_size >= kMaxDim || num_pages * page_size >= kMaxDim)
    return fail(MQ_ERR_INVALID, "[%s] the page table is too large (2^31 slots at most).", op);
  return MQ_OK;
}
}  // namespace

int mq_rope_kv_append(const mq_bf16* qkv, const int64_t* positions, const int32_t* page_table,
                      int64_t pages_per_seq, int64_t page_size, int64_t num_pages,
                      const float* cos_table, const float* sin_table, const mq_bf16* q_norm,
                      const mq_bf16* k_norm, float norm_eps, mq_bf16* q_out, mq_bf16* k_pages,
                      mq_bf16* v_pages, int64_t batch, int n_heads, int n_kv_heads, int head_dim,
                      hipStream_t stream) {
  const char* op = "rope_kv_append";
  if (int rc = check_pages(op, batch, n_heads, n_kv_heads, pages_per_seq, page_size, num_pages))
    return rc;
  if (head_dim <= 0 || head_dim % 2)
    return fail(MQ_ERR_INVALID, "[%s] head_dim=%d must be even.", op, head_dim);
  if ((q_norm || k_norm) && head_dim > 128)
    return fail(MQ_ERR_UNSUPPORTED, "[%s] q/k norms need head_dim <= 128, got %d.", op,
                head_dim);
  if (batch == 0) return ok();
  if (!qkv || !positions || !page_table || !cos_table || !sin_table || !q_out || !k_pages ||
      !v_pages)
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  return hip_status(mq::launch_rope_append(qkv, positions, page_table, pages_per_seq, page_size,
                                           num_pages, q_norm, k_norm, norm_eps, cos_table,
                                           sin_table, q_out, k_pages, v_pages, batch, n_heads,
                                           n_kv_heads, head_dim, stream),
                    op);
}

size_t mq_paged_decode_attention_workspace(int64_t batch, int n_heads, int n_kv_heads,
                                           int head_dim, int64_t pages_per_seq,
                                           int64_t page_size) {
  if (batch <= 0 || batch > 65535 || pages_per_seq <= 0 || page_size <= 0 ||
      pages_per_seq * page_size >= kMaxDim ||
      !mq::decode_attention_supported(n_heads, n_kv_heads, head_dim))
    return 0;
  return mq::decode_attention_workspace(batch, n_heads, n_kv_heads, head_dim,
                                        pages_per_seq * page_size);
}

int mq_paged_decode_attention(const mq_bf16* q, const mq_bf16* k_pages, const mq_bf16* v_pages,
                              const int32_t* page_table, int64_t pages_per_seq, int64_t page_size,
                              int64_t num_pages, const int64_t* positions, int64_t batch,
                              int n_heads, int n_kv_heads, int head_dim, float scale,
                              void* workspace, size_t workspace_bytes, mq_bf16* out,
                              hipStream_t stream) {
  const char* op = "paged_decode_attention";
  if (int rc = check_pages(op, batch, n_heads, n_kv_heads, pages_per_seq, page_size, num_pages))
    return rc;
  if (!mq::decode_attention_supported(n_heads, n_kv_heads, head_dim))
    return fail(MQ_ERR_UNSUPPORTED,
                "[%s] head_dim=%d with %d query heads per KV head is not supported (64 or 128; "
                "1-8).",
                op, head_dim, n_kv_heads > 0 ? n_heads / n_kv_heads : 0);
  if (batch == 0) return ok();
  const size_t need = mq::decode_attention_workspace(batch, n_heads, n_kv_heads, head_dim,
                                                     pages_per_seq * page_size);
  if (!workspace || workspace_bytes < need)
    return fail(MQ_ERR_INVALID, "[%s] the workspace needs %zu bytes, got %zu.", op, need,
                workspace ? workspace_bytes : (size_t)0);
  if (!q || !k_pages || !v_pages || !page_table || !positions || !out)
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(q) || !aligned16(k_pages) || !aligned16(v_pages) || !aligned16(workspace))
    return fail(MQ_ERR_INVALID, "[%s] q, the pages and the workspace must be 16-byte aligned.",
                op);
  return hip_status(mq::launch_decode_attention(q, k_pages, v_pages, page_table, pages_per_seq,
                                                page_size, num_pages, positions, batch, n_heads,
                                                n_kv_heads, head_dim, scale,
                                                static_cast<float*>(workspace), out, stream),
                    op);
}

int mq_decode_attention_step(const mq_bf16* qkv, const int64_t* positions,
                             const int32_t* page_table, int64_t pages_per_seq, int64_t page_size,
                             int64_t num_pages, const float* cos_table, const float* sin_table,
                             const mq_bf16* q_norm, const mq_bf16* k_norm, float norm_eps,
                             mq_bf16* k_pages, mq_bf16* v_pages, int64_t batch, int n_heads,
                             int n_kv_heads, int head_dim, float scale, void* workspace,
                             size_t workspace_bytes, mq_bf16* out, hipStream_t stream) {
  const char* op = "decode_attention_step";
  if (int rc = check_pages(op, batch, n_heads, n_kv_heads, pages_per_seq, page_size, num_pages))
    return rc;
  if (!mq::decode_attention_supported(n_heads, n_kv_heads, head_dim))
    return fail(MQ_ERR_UNSUPPORTED,
                "[%s] head_dim=%d with %d query heads per KV head is not supported (64 or 128; "
                "1-8).",
                op, head_dim, n_kv_heads > 0 ? n_heads / n_kv_heads : 0);
  if (batch == 0) return ok();
  const size_t need = mq::decode_attention_workspace(batch, n_heads, n_kv_heads, head_dim,
                                                     pages_per_seq * page_size);
  if (!workspace || workspace_bytes < need)
    return fail(MQ_ERR_INVALID, "[%s] the workspace needs %zu bytes, got %zu.", op, need,
                workspace ? workspace_bytes : (size_t)0);
  if (!qkv || !positions || !page_table || !cos_table || !sin_table || !k_pages || !v_pages ||
      !out)
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(qkv) || !aligned16(k_pages) || !aligned16(v_pages) || !aligned16(workspace))
    return fail(MQ_ERR_INVALID, "[%s] qkv, the pages and the workspace must be 16-byte aligned.",
                op);
  return hip_status(mq::launch_attention_step(qkv, positions, page_table, pages_per_seq,
                                              page_size, num_pages, cos_table, sin_table, q_norm,
                                              k_norm, norm_eps, k_pages, v_pages, batch, n_heads,
                                              n_kv_heads, head_dim, scale,
                                              static_cast<float*>(workspace), out, stream),
                    op);
}

int mq_paged_prefill_attention_supported(int n_heads, int n_kv_heads, int head_dim,
                                         int64_t num_pages, int64_t page_size) {
  return n_heads > 0 && n_heads <= 65535 && n_kv_heads > 0 && n_heads % n_kv_heads == 0 &&
                 num_pages > 0 && page_size > 0 &&
                 mq::prefill_attention_supported(n_heads, n_kv_heads, head_dim, num_pages,
                                                 page_size)
             ? 1
             : 0;
}

int mq_paged_prefill_attention(const mq_bf16* q, const mq_bf16* k_pages, const mq_bf16* v_pages,
                               const int32_t* page_table, int64_t pages_per_seq,
                               int64_t page_size, int64_t num_pages, const int64_t* starts,
                               const int64_t* lens, int64_t batch, int64_t tokens, int n_heads,
                               int n_kv_heads, int head_dim, float scale, mq_bf16* out,
                               hipStream_t stream) {
  const char* op = "paged_prefill_attention";
  if (int rc = check_pages(op, batch, n_heads, n_kv_heads, pages_per_seq, page_size, num_pages))
    return rc;
  if (int rc = check_dim(op, "tokens", tokens)) return rc;
  if (n_heads > 65535)
    return fail(MQ_ERR_UNSUPPORTED, "[%s] n_heads=%d > 65535.", op, n_heads);
  if (!mq::prefill_attention_supported(n_heads, n_kv_heads, head_dim, num_pages, page_size))
    return fail(MQ_ERR_UNSUPPORTED,
                "[%s] head_dim=%d is not supported (128), or the pages of one layer exceed 2 GiB.",
                op, head_dim);
  if (batch == 0 || tokens == 0) return ok();
  if (batch * tokens * n_heads * (int64_t)head_dim >= kMaxDim * (int64_t)64)
    return fail(MQ_ERR_INVALID, "[%s] q is too large.", op);
  if (!q || !k_pages || !v_pages || !page_table || !starts || !lens || !out)
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(q) || !aligned16(k_pages) || !aligned16(v_pages))
    return fail(MQ_ERR_INVALID, "[%s] q and the pages must be 16-byte aligned.", op);
  return hip_status(mq::launch_prefill_attention(q, k_pages, v_pages, page_table, pages_per_seq,
                                                 page_size, num_pages, starts, lens, batch,
                                                 tokens, n_heads, n_kv_heads, scale, out, stream),
                    op);
}

int mq_silu_mul(const mq_bf16* gate_up, mq_bf16* out, int64_t rows, int64_t inter,
                hipStream_t stream) {
  const char* op = "silu_mul";
  if (int rc = check_dim(op, "rows", rows)) return rc;
  if (inter <= 0 || inter % 8 || inter >= kMaxDim)
    return fail(MQ_ERR_UNSUPPORTED, "[%s] the width %lld must be a positive multiple of 8.", op,
                (long long)inter);
  if (rows == 0) return ok();
  if (!gate_up || !out) return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(gate_up) || !aligned16(out))
    return fail(MQ_ERR_INVALID, "[%s] buffers must be 16-byte aligned.", op);
  return hip_status(mq::launch_silu_mul(gate_up, out, rows, inter, stream), op);
}

int mq_moe_route(const mq_bf16* logits, const float* expert_bias, int64_t tokens,
                 int num_experts, int top_k, int norm_topk_prob, int32_t* indices,
                 mq_bf16* scores, hipStream_t stream) {
  const char* op = "moe_route";
  if (int rc = check_dim(op, "tokens", tokens)) return rc;
  if (!mq::moe_route_supported(num_experts, top_k))
    return fail(MQ_ERR_UNSUPPORTED, "[%s] %d experts, top %d: 1 <= k <= min(E, 64), E <= 512.",
                op, num_experts, top_k);
  if (tokens == 0) return ok();
  if (!logits || !indices || !scores) return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  return hip_status(mq::launch_moe_route(logits, expert_bias, tokens, num_experts, top_k,
                                         norm_topk_prob != 0, indices, scores, stream),
                    op);
}

int mq_moe_sort(const int32_t* expert_ids, int64_t n, int top_k, int num_experts,
                int32_t* sorted_ids, int32_t* order, int32_t* inverse, int32_t* rows,
                int32_t* expert_offsets, hipStream_t stream) {
  const char* op = "moe_sort";
  if (int rc = check_dim(op, "n", n)) return rc;
  if (top_k < 1) return fail(MQ_ERR_INVALID, "[%s] top_k=%d must be >= 1.", op, top_k);
  if (!mq::moe_sort_supported(n, num_experts))
    return fail(MQ_ERR_UNSUPPORTED, "[%s] %d experts (1..512), %lld entries (< 2^30).", op,
                num_experts, (long long)n);
  if (n == 0 && !expert_offsets) return ok();
  if (n > 0 && (!expert_ids || !sorted_ids || !order || !inverse))
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  return hip_status(mq::launch_moe_sort(expert_ids, n, top_k, num_experts, sorted_ids, order,
                                        inverse, rows, expert_offsets, stream),
                    op);
}

int mq_moe_combine(const mq_bf16* y, const int32_t* inverse, const mq_bf16* scores, mq_bf16* out,
                   int64_t tokens, int top_k, int64_t hidden, hipStream_t stream) {
  const char* op = "moe_combine";
  if (int rc = check_dim(op, "tokens", tokens)) return rc;
  if (top_k < 1 || (int64_t)top_k * tokens >= kMaxDim)
    return fail(MQ_ERR_INVALID, "[%s] top_k=%d is out of range.", op, top_k);
  if (hidden <= 0 || hidden % 8 || hidden >= kMaxDim)
    return fail(MQ_ERR_UNSUPPORTED, "[%s] hidden=%lld must be a positive multiple of 8.", op,
                (long long)hidden);
  if (tokens == 0) return ok();
  if (!y || !scores || !out) return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(y) || !aligned16(out))
    return fail(MQ_ERR_INVALID, "[%s] y and out must be 16-byte aligned.", op);
  return hip_status(mq::launch_moe_combine(y, inverse, scores, out, tokens, top_k, hidden, stream),
                    op);
}

int mq_moe_route_sort(const mq_bf16* logits, const float* expert_bias, int64_t tokens,
                      int num_experts, int top_k, int norm_topk_prob, int32_t* indices,
                      mq_bf16* scores, int32_t* sorted_ids, int32_t* order, int32_t* inverse,
                      int32_t* rows, int32_t* expert_offsets, hipStream_t stream) {
  const char* op = "moe_route_sort";
  if (int rc = check_dim(op, "tokens", tokens)) return rc;
  if (!mq::moe_route_supported(num_experts, top_k))
    return fail(MQ_ERR_UNSUPPORTED, "[%s] %d experts, top %d: 1 <= k <= min(E, 64), E <= 512.",
                op, num_experts, top_k);
  if (!mq::moe_sort_supported(tokens * top_k, num_experts))
    return fail(MQ_ERR_UNSUPPORTED, "[%s] %lld entries (< 2^30).", op,
                (long long)(tokens * top_k));
  if (tokens == 0)
    return expert_offsets ? mq_moe_sort(nullptr, 0, top_k, num_experts, nullptr, nullptr,
                                        nullptr, nullptr, expert_offsets, stream)
                          : ok();
  if (!logits || !indices || !scores || !sorted_ids || !order || !inverse)
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  return hip_status(mq::launch_moe_route_sort(logits, expert_bias, tokens, num_experts, top_k,
                                              norm_topk_prob != 0, indices, scores, sorted_ids,
                                              order, inverse, rows, expert_offsets, stream),
                    op);
}

int mq_argmax_rows(const mq_bf16* x, int64_t rows, int64_t cols, int64_t* out,
                   hipStream_t stream) {
  const char* op = "argmax_rows";
  if (int rc = check_dim(op, "rows", rows)) return rc;
  // a row's byte offsets are 32-bit: at most 2^28 elements
  if (cols < 1 || cols > ((int64_t)1 << 28))
    return fail(MQ_ERR_INVALID, "[%s] cols=%lld is out of range (1..2^28).", op,
                (long long)cols);
  if (cols % 8)
    return fail(MQ_ERR_UNSUPPORTED, "[%s] cols=%lld: rows of whole 8-element units only.", op,
                (long long)cols);
  if (rows == 0) return ok();
  if (!x || !out) return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(x)) return fail(MQ_ERR_INVALID, "[%s] x must be 16-byte aligned.", op);
  return hip_status(mq::launch_argmax_rows(x, rows, cols, out, stream), op);
}

int mq_moe_combine_rms_norm(const mq_bf16* y, const int32_t* inverse, const mq_bf16* scores,
                            const mq_bf16* residual, mq_bf16* residual_out,
                            const mq_bf16* weight, mq_bf16* out, int64_t tokens, int top_k,
                            int64_t hidden, float eps, hipStream_t stream) {
  const char* op = "moe_combine_rms_norm";
  if (int rc = check_dim(op, "tokens", tokens)) return rc;
  if (top_k < 1 || (int64_t)top_k * tokens >= kMaxDim)
    return fail(MQ_ERR_INVALID, "[%s] top_k=%d is out of range.", op, top_k);
  if (!mq::moe_combine_norm_supported(hidden))
    return fail(MQ_ERR_UNSUPPORTED, "[%s] hidden=%lld is not supported (a multiple of 8, <= 8192).",
                op, (long long)hidden);
  if (tokens == 0) return ok();
  if (!y || !scores || !residual || !residual_out || !weight || !out)
    return fail(MQ_ERR_INVALID, "[%s] null pointer.", op);
  if (!aligned16(y) || !aligned16(residual) || !aligned16(residual_out) || !aligned16(weight) ||
      !aligned16(out))
    return fail(MQ_ERR_INVALID, "[%s] y, residual, residual_out, weight and out must be 16-byte "
                "aligned.", op);
  return hip_status(mq::launch_moe_combine_norm(y, inverse, scores, residual, residual_out, weight,
                                                out, tokens, top_k, hidden, eps, stream),
                    op);
}

}  // extern "C"
