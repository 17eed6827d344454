// Launchers shared between the kernel translation units and the C-ABI.
// Every launcher assumes its arguments were validated by the C-ABI layer
// (mq_capi.hip) and only enqueues work on `stream`.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mq {

// Sets the calling thread's mq_last_error() message; returns code.  For
// entry points defined outside mq_capi.hip.
int set_last_error(int code, const char* msg);

struct GatherMap {
  const int32_t* lhs;   // x batch per output batch (nullptr: identity)
  const int32_t* rhs;   // expert per output batch (nullptr: single matrix)
  int64_t T;            // output batches (1 for a plain matmul)
  int64_t E;            // experts
  int64_t x_batches;    // batches in x
};

// Group sizes 32, 64 and 128 (K a multiple of the group size).
hipError_t launch_quantize(const uint16_t* w, uint32_t* wq, uint16_t* scales, uint16_t* biases,
                           int64_t rows, int64_t K, int group_size, int bits, hipStream_t stream);
hipError_t launch_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                             const int32_t* row_ids, int64_t n_out_rows, int64_t n_rows,
                             uint16_t* out, int64_t K, int group_size, int bits,
                             hipStream_t stream);
// 2/3/5/6-bit stream codes [rows, K * bits / 32] -> one byte per code
// [rows, K / 4] (the 8-bit layout; same scales and biases).
hipError_t launch_repack_u8(const uint32_t* wq, uint32_t* wq8, int64_t rows, int64_t K, int bits,
                            hipStream_t stream);

// y[t][m][n] = x[lhs[t]][m] . dequant(w[rhs[t]][n]) (+ bias[n]); valid when
// qmv_fits(M, N, K, bits, T, group_size) (at most 8 rows, x and the scales
// staged within the LDS budget; group size 32, 64 or 128).
bool qmv_fits(int64_t M, int64_t N, int64_t K, int bits, int64_t T, int group_size);
hipError_t launch_qmv(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                      const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                      int64_t N, int64_t K, int bits, const GatherMap& g, int group_size,
                      hipStream_t stream);
// Gathered SwiGLU GEMV: y [T, M, N] per (batch, expert) pair of g; every
// expert's matrix is 2N rows (gate rows, then up rows).
bool gather_qmv_swiglu_fits(int64_t M, int64_t N, int64_t K, int bits, int64_t T,
                            int group_size);
hipError_t launch_gather_qmv_swiglu(const uint16_t* x, const uint32_t* wq,
                                    const uint16_t* scales, const uint16_t* biases, uint16_t* y,
                                    int64_t M, int64_t N, int64_t K, int bits, const GatherMap& g,
                                    int group_size, hipStream_t stream);
bool qmv_swiglu_fits(int64_t M, int64_t N, int64_t K, int bits, int group_size);
bool qmv_norm_fits(int64_t N, int64_t K, int bits, bool swiglu, int group_size);
hipError_t launch_qmv_norm(const uint16_t* a, const uint16_t* res, uint16_t* res_out,
                           const uint16_t* norm_w, float eps, const uint32_t* wq,
                           const uint16_t* scales, const uint16_t* biases, const uint16_t* bias,
                           uint16_t* y, int64_t N, int64_t K, int bits, bool swiglu,
                           int group_size, hipStream_t stream);
hipError_t launch_qmv_swiglu(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                             const uint16_t* biases, uint16_t* y, int64_t M, int64_t N, int64_t K,
                             int bits, int group_size, hipStream_t stream);

// The one-row 4-bit GEMV for rows of 16 lanes (K a multiple of 512, 1024 to
// 4096, group size 32, 64 or 128): where qmv1_fits(M, rows, K, bits,
// group_size) holds (rows: 2N with swiglu), mq_quantized_matmul and the
// SwiGLU / RMSNorm fused entries run it (bit-identical to qmv_kernel where
// that runs 16 lanes per row).
namespace qmv {
struct NormIn;
}
bool qmv1_fits(int64_t M, int64_t rows, int64_t K, int bits, int group_size);
// ... and where its plain form (no SwiGLU, no RMSNorm input) runs: also the
// long rows of down projections.
bool qmv1_plain_fits(int64_t M, int64_t rows, int64_t K, int bits, int group_size);
// The same kernel's plain form on 2, 3, 5 or 6-bit codes read at their width
// (a 32-code chunk is `bits` whole words of the row's bit stream): one row,
// the K values of qmv1_plain_fits.
bool qmvs_fits(int64_t M, int64_t rows, int64_t K, int bits, int group_size);
hipError_t launch_qmvs(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t N,
                       int64_t K, int bits, int group_size, hipStream_t stream);
hipError_t launch_qmv1(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t N,
                       int64_t K, int group_size, bool swiglu, const qmv::NormIn* nrm,
                       hipStream_t stream);

// Same contract on the matrix cores for M <= 8 (4-bit) / 16 (8-bit); valid
// when qmvm_fits(M, N, K, bits, T) (K a multiple of 256, at most 12 chunks
// per lane).
bool qmvm_fits(int64_t M, int64_t N, int64_t K, int bits, int64_t T);
hipError_t launch_qmvm(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                       int64_t N, int64_t K, int bits, const GatherMap& g, hipStream_t stream);

// 256x256-tile MFMA path with weights dequantized in registers (qmm4_fits:
// group size 32, 64 or 128, K an even number of groups, >= 128 tiles or few
// tiles with K splits, 32-bit offsets), two waves per SIMD, each owning the block's 256 rows for
// 32 columns (every code dequantized once per block).  Few tiles and a long
// K: K is split over blocks; a short last round of tiles: those tiles go to
// stream-K blocks (qmm4_stream_k).  Both write float32 partial sums to a
// workspace of qmm4_workspace_bytes; without it every tile runs whole.
// qmm4_unsplit: the plan splits no tile's K evenly (the SwiGLU form's plan).
bool qmm4_fits(int64_t M, int64_t N, int64_t K, int bits, int group_size);
size_t qmm4_workspace_bytes(int64_t M, int64_t N, int64_t K, int group_size);
bool qmm4_unsplit(int64_t M, int64_t N, int64_t K, int group_size);
bool qmm4_stream_k(int64_t M, int64_t N, int64_t K, int group_size);
// mq_quantized_matmul_ws takes the shape with less workspace than it asks for
// (mq_capi.hip).
bool qmm_workspace_optional(int64_t M, int64_t N, int64_t K, int group_size, int bits);
hipError_t launch_qmm4(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                       int64_t N, int64_t K, int bits, int group_size, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);
// The same kernel over rows sorted by expert (gather_qmm with sorted
// indices): rows = T * Mb, row p = (batch p / Mb, row p % Mb) reads x batch
// lhs[batch] (the batch itself without lhs) and expert rhs[batch]; tiles are
// 256-row pieces of one expert's segment.  seg (E + 1 batch offsets of the
// segments) or, when null, a scan of rhs (non-decreasing) gives the segments;
// rows whose id names no expert are zero.  swiglu: every expert's matrix is
// 2N rows (gate, then up) and y [T*Mb, N] = silu(gate) * up.
bool qmm4_gather_fits(int64_t T, int64_t Mb, int64_t N, int64_t K, int64_t E,
                      int64_t x_batches, int bits, int group_size);
hipError_t launch_qmm4_gather(const uint16_t* x, const int32_t* lhs, const int32_t* rhs,
                              const int32_t* seg, const uint32_t* wq, const uint16_t* scales,
                              const uint16_t* biases, uint16_t* y, int64_t T, int64_t Mb,
                              int64_t N, int64_t K, int64_t E, int64_t x_batches, int bits,
                              int group_size, bool swiglu, hipStream_t stream);
// The dense kernel on a gate|up matrix [2N, K] (gate rows first) with
// silu(gate) * up in its epilogue: y [M, N] (unsplit launches only).
bool qmm4_swiglu_fits(int64_t M, int64_t N, int64_t K, int bits, int group_size);
hipError_t launch_qmm4_swiglu(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                              const uint16_t* biases, uint16_t* y, int64_t M, int64_t N,
                              int64_t K, int bits, int group_size, hipStream_t stream);
// y[i] = bf16(sum over s < splits of partial[s * MN + i] (in order) + bias[i % N])
hipError_t launch_splitk_reduce(const float* partial, int splits, const uint16_t* bias,
                                uint16_t* y, int64_t MN, int64_t N, hipStream_t stream);

// Skinny MFMA path (M up to a few hundred): weights streamed once per M tile
// of up to 128 rows; K split over blocks through a float32 workspace when the
// tiles alone cannot fill the GPU (qmms_workspace_bytes > 0).  Without a large
// enough workspace it runs unsplit.  Group sizes 32, 64 and 128 (the plans do
// not depend on it).
bool qmms_fits(int64_t M, int64_t N, int64_t K, int bits);
size_t qmms_workspace_bytes(int64_t M, int64_t N, int64_t K, int bits);
// Split plans of the skinny GEMM whose reduce can take an epilogue: SwiGLU of
// a [2 Nout, K] gate|up matrix, or + residual and RMSNorm (N <= 8192).
bool qmms_split_fusable(int64_t M, int64_t N, int64_t K, int bits);
// The skinny GEMM's unsplit one-tile plan for a 2*Nout-row gate|up matrix,
// with silu(gate) * up in its epilogue.
bool qmms_swiglu_direct(int64_t M, int64_t Nout, int64_t K, int bits);
hipError_t launch_qmms_swiglu_direct(const uint16_t* x, const uint32_t* wq,
                                     const uint16_t* scales, const uint16_t* biases, uint16_t* y,
                                     int64_t M, int64_t Nout, int64_t K, int bits,
                                     int group_size, hipStream_t stream);
hipError_t launch_qmms_swiglu(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                              const uint16_t* biases, uint16_t* y, int64_t M, int64_t Nout,
                              int64_t K, int bits, int group_size, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);
hipError_t launch_qmms_add_norm(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                                const uint16_t* biases, const uint16_t* bias,
                                const uint16_t* residual, uint16_t* residual_out,
                                const uint16_t* norm_w, float eps, uint16_t* out, int64_t M,
                                int64_t N, int64_t K, int bits, int group_size, void* workspace,
                                size_t workspace_bytes, hipStream_t stream);
hipError_t launch_qmms(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                       int64_t N, int64_t K, int bits, int group_size, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);

// MFMA path, any M, group size 32, 64 or 128.
hipError_t launch_qmm(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                      const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                      int64_t N, int64_t K, int group_size, int bits, hipStream_t stream);
// MFMA gather over flattened rows r = t*rows_per_batch + m: x row
// lhs[t]*rows_per_batch + m (x_rows rows in x) times expert rhs[t]; the rows of
// one expert inside a row tile share one pass over the weights.
hipError_t launch_gather_qmm_rows(const uint16_t* x, const int32_t* lhs, const int32_t* rhs,
                                  const uint32_t* wq, const uint16_t* scales,
                                  const uint16_t* biases, uint16_t* y, int64_t rows, int64_t N,
                                  int64_t K, int64_t E, int64_t x_rows, int rows_per_batch,
                                  int group_size, int bits, hipStream_t stream);

// Decoder-step kernels (mq_decoder.hip).  KV pages: bfloat16
// [num_pages, page_size, nkv, head_dim]; page table int32 [B, pages_per_seq];
// pos int64 [B] is the position of each sequence's current token.
bool rmsnorm_supported(int64_t dim);
hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* res_in, uint16_t* res_out,
                          const uint16_t* w, uint16_t* out, int64_t rows, int64_t dim, float eps,
                          hipStream_t stream);
hipError_t launch_rope_append(const uint16_t* qkv, const int64_t* pos, const int32_t* page_table,
                              int64_t pages_per_seq, int64_t page_size, int64_t num_pages,
                              const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                              const float* cos_t, const float* sin_t, uint16_t* q_out,
                              uint16_t* k_pages, uint16_t* v_pages, int64_t B, int nh, int nkv,
                              int d, hipStream_t stream);
bool decode_attention_supported(int nh, int nkv, int d);
size_t decode_attention_workspace(int64_t B, int nh, int nkv, int d, int64_t capacity);
hipError_t launch_decode_attention(const uint16_t* q, const uint16_t* k_pages,
                                   const uint16_t* v_pages, const int32_t* page_table,
                                   int64_t pages_per_seq, int64_t page_size, int64_t num_pages,
                                   const int64_t* pos, int64_t B, int nh, int nkv, int d,
                                   float scale, float* workspace, uint16_t* out,
                                   hipStream_t stream);
// out int64 [rows] = the first index of each bfloat16 row's largest value
// (cols % 8 == 0, x 16-byte aligned; NaN counts as the largest).
hipError_t launch_argmax_rows(const uint16_t* x, int64_t rows, int64_t cols, int64_t* out,
                              hipStream_t stream);
hipError_t launch_silu_mul(const uint16_t* gu, uint16_t* out, int64_t rows, int64_t inter,
                           hipStream_t stream);
// RoPE + append fused into the split attention kernel, then the combine.
hipError_t launch_attention_step(const uint16_t* qkv, const int64_t* pos,
                                 const int32_t* page_table, int64_t pages_per_seq,
                                 int64_t page_size, int64_t num_pages, const float* cos_t,
                                 const float* sin_t, const uint16_t* q_norm,
                                 const uint16_t* k_norm, float eps, uint16_t* k_pages,
                                 uint16_t* v_pages, int64_t B, int nh, int nkv, int d,
                                 float scale, float* workspace, uint16_t* out,
                                 hipStream_t stream);

// Paged causal attention of prefill chunks (mq_prefill_attn.hip).
bool prefill_attention_supported(int nh, int nkv, int d, int64_t num_pages, int64_t page_size);
hipError_t launch_prefill_attention(const uint16_t* q, const uint16_t* k_pages,
                                    const uint16_t* v_pages, const int32_t* page_table,
                                    int64_t pages_per_seq, int64_t page_size, int64_t num_pages,
                                    const int64_t* starts, const int64_t* lens, int64_t B,
                                    int64_t T, int nh, int nkv, float scale, uint16_t* out,
                                    hipStream_t stream);

// Mixture-of-experts routing (mq_moe.hip).
bool moe_route_supported(int E, int k);
hipError_t launch_moe_route(const uint16_t* logits, const float* expert_bias, int64_t T, int E,
                            int k, bool normalize, int32_t* indices, uint16_t* scores,
                            hipStream_t stream);
bool moe_sort_supported(int64_t n, int E);
hipError_t launch_moe_sort(const int32_t* ids, int64_t n, int k, int E, int32_t* sorted_ids,
                           int32_t* order, int32_t* inverse, int32_t* rows,
                           int32_t* expert_offsets, hipStream_t stream);
hipError_t launch_moe_combine(const uint16_t* y, const int32_t* inverse, const uint16_t* scores,
                              uint16_t* out, int64_t T, int k, int64_t H, hipStream_t stream);
hipError_t launch_moe_route_sort(const uint16_t* logits, const float* expert_bias, int64_t T,
                                 int E, int k, bool normalize, int32_t* indices, uint16_t* scores,
                                 int32_t* sorted_ids, int32_t* order, int32_t* inverse,
                                 int32_t* rows, int32_t* expert_offsets, hipStream_t stream);
bool moe_combine_norm_supported(int64_t H);
hipError_t launch_moe_combine_norm(const uint16_t* y, const int32_t* inverse,
                                   const uint16_t* scores, const uint16_t* residual,
                                   uint16_t* residual_out, const uint16_t* w, uint16_t* normed,
                                   int64_t T, int k, int64_t H, float eps, hipStream_t stream);

}  // namespace mq
