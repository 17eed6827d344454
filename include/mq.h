/*
 * mq.h -- C ABI of libmi355q, the MI355X (gfx950) affine-quantized matmul path.
 *
 * Drop-in boundary for the quantized linear layers of the reference's native
 * MLX worker (huydt84/mlx-server-runtime, python/mlx_worker/native_mlx/).  The
 * reference reaches this path only through the Python API of the external mlx
 * 0.31.2 package (python/uv.lock:939-941); each entry point below replaces one
 * of those calls, with the same tensors and the same argument meaning.
 *
 * Conventions
 *   - All array pointers are DEVICE pointers owned by the caller; the library
 *     allocates nothing and never synchronizes the host.  Work is enqueued on
 *     `stream` (NULL = the default stream).
 *   - bfloat16 data is passed as raw 16-bit patterns (mq_bf16).
 *   - Weight format (MLX "affine"): wq uint32 [rows, K*bits/32] with codes
 *     packed LSB-first as one bit stream per row (code k at bits
 *     [k*bits, (k+1)*bits) of the row's words: 32/bits codes per word for 2,
 *     4 and 8 bits; for 3, 5 and 6 bits MLX's 8, 8 and 4 codes per 3, 5 and
 *     3 bytes, a code possibly straddling two words); scales and biases
 *     bfloat16 [rows, K/group_size]; w = scale*q + bias.
 *   - Supported here: bits 2, 3, 4, 5, 6 and 8 with group_size 32, 64 or 128
 *     for mq_quantize, mq_dequantize and mq_embedding_lookup.  At 2/3/5/6
 *     bits mq_quantized_matmul[_ws] reads one-row products' codes at their
 *     width (K a multiple of 512 from 1024 to 4096, or 13824/14336/18944 at
 *     group size 64/128: no workspace); other shapes it runs by rewriting
 *     the codes one byte each into its workspace
 *     (mq_quantized_matmul_workspace counts those bytes) and running the
 *     8-bit kernels with the same scales and biases.  The other matmul entry
 *     points read 4- and 8-bit codes and return MQ_ERR_UNSUPPORTED for the
 *     rest (mq_repack_codes_u8 converts a matrix once, e.g. at load time,
 *     to call them with bits = 8).  transpose
 *     = 0 returns MQ_ERR_UNSUPPORTED; anything MLX itself rejects returns
 *     MQ_ERR_INVALID.
 *     Every matmul entry point, fused ones included, takes group sizes 32,
 *     64 and 128 (the *_supported queries answer for each); a matmul of more
 *     than 8 rows with group_size 32 needs K to be a multiple of 64 (else
 *     MQ_ERR_UNSUPPORTED).
 *   - Pointers that feed 16-byte loads (x, wq, w, out, y rows) must be 16-byte
 *     aligned.
 *   - Return value: MQ_OK, or a negative code with a message available from
 *     mq_last_error() on the calling thread.  Validation happens before any
 *     launch, so a failed call enqueues nothing.
 *   - Reentrant: no mutable global state besides the thread-local message
 *     (and mq_quantized_matmul_noalloc's per-GPU array, see there).
 */
#ifndef MQ_H
#define MQ_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t mq_bf16; /* raw bfloat16 bits */

#define MQ_OK 0
#define MQ_ERR_INVALID (-1)     /* arguments MLX would reject too */
#define MQ_ERR_UNSUPPORTED (-2) /* valid for MLX, not implemented here */
#define MQ_ERR_HIP (-3)         /* the HIP runtime refused a launch */

/* (major << 16) | minor.  2.0: mq_moe_sort and mq_moe_route_sort take an
 * expert_offsets output before the stream argument (1.0 had none).  2.1 adds
 * mq_paged_prefill_attention and its _supported query, 2.2 mq_argmax_rows. */
int mq_version(void);

/* Message for the last failed call on this thread ("" if none). */
const char* mq_last_error(void);

/*
 * mx.quantize(w, group_size, bits, mode="affine") for bfloat16 w [rows, K]:
 * writes wq [rows, K*bits/32], scales and biases [rows, K/group_size].
 * Replaces the calls at python/mlx_worker/native_mlx/models/lfm2.py:112-117
 * and :142-151 and the one nn.quantize makes per layer
 * (models/qwen2.py:318-324).  Bit-exact with the float32 algorithm.
 */
int mq_quantize(const mq_bf16* w, uint32_t* wq, mq_bf16* scales, mq_bf16* biases, int64_t rows,
                int64_t K, int group_size, int bits, hipStream_t stream);

/*
 * mx.dequantize(wq, scales, biases, group_size, bits) -> out bfloat16 [rows, K],
 * out = bf16(bf16(q*scale) + bias).
 */
int mq_dequantize(const uint32_t* wq, const mq_bf16* scales, const mq_bf16* biases, mq_bf16* out,
                  int64_t rows, int64_t K, int group_size, int bits, hipStream_t stream);

/*
 * Quantized embedding lookup: out[i] = dequantize(wq[ids[i]]) for i < n_ids,
 * the nn.QuantizedEmbedding call behind models/qwen2.py:185 (embed_tokens).
 * An id outside [0, rows) yields a row of zeros.
 */
int mq_embedding_lookup(const int32_t* ids, int64_t n_ids, const uint32_t* wq,
                        const mq_bf16* scales, const mq_bf16* biases, int64_t rows, int64_t K,
                        int group_size, int bits, mq_bf16* out, hipStream_t stream);

/*
 * 2/3/5/6-bit codes wq [rows, K*bits/32] -> the same codes one byte each,
 * wq8 [rows, K/4] (the 8-bit layout): with the unchanged scales and biases
 * the matrix dequantizes to the same weights and runs on every 8-bit entry
 * point.  No counterpart in MLX (its kernels read these widths directly); it
 * is the load-time step a caller takes where a checkpoint's config.json
 * "quantization" gives such bits for a path (models/qwen2.py:316-324,
 * models/lfm2.py:579-589).  K a multiple of 32; wq8 16-byte aligned.
 */
int mq_repack_codes_u8(const uint32_t* wq, uint32_t* wq8, int64_t rows, int64_t K, int bits,
                       hipStream_t stream);

/*
 * mx.quantized_matmul(x, wq, scales, biases, transpose=True, group_size, bits)
 * plus QuantizedLinear's optional "+ bias":
 *   y[m, n] = sum_k x[m, k] * (scale*q + bias)[n, k]  (+ bias_vec[n])
 * x bfloat16 [M, K], wq [N, K*bits/32], bias_vec bfloat16 [N] or NULL,
 * y bfloat16 [M, N]; float32 accumulation, one rounding at the store.
 * Replaces every QuantizedLinear call of the model graphs
 * (models/qwen2.py:76-78,115,134,227; qwen3.py:78-86,115,134,222).
 * Decode-sized M uses the GEMV kernels, larger M the MFMA kernels; this
 * entry point never splits K (see mq_quantized_matmul_ws).
 */
int mq_quantized_matmul(const mq_bf16* x, const uint32_t* wq, const mq_bf16* scales,
                        const mq_bf16* biases, const mq_bf16* bias_vec, mq_bf16* y, int64_t M,
                        int64_t N, int64_t K, int group_size, int bits, int transpose,
                        hipStream_t stream);

/*
 * Workspace, in bytes, that mq_quantized_matmul_ws can use for this shape
 * (0 = none).  Shapes whose output tiles cannot fill the GPU and have a long
 * K (the down projection at small M, and at M = 1-2K prefill chunks) split K
 * over blocks and need float32 partial sums; so do large-M shapes whose
 * 256 x 256 tiles leave a short last round of the GPU (at most 85 of 256
 * tiles): those tiles run as stream-K pieces.
 * MLX allocates such temporaries internally; this library allocates nothing,
 * so the caller provides them.  No counterpart in the reference: it serves
 * the same mx.quantized_matmul call sites as mq_quantized_matmul.
 */
size_t mq_quantized_matmul_workspace(int64_t M, int64_t N, int64_t K, int group_size, int bits);

/*
 * mq_quantized_matmul with a caller-owned device workspace (16-byte aligned,
 * `workspace_bytes` long; NULL/0 allowed).  With at least
 * mq_quantized_matmul_workspace() bytes, K may be split over blocks; with
 * less it runs unsplit (every large-M tile whole).  Results are identical run
 * to run either way (the partial sums are added in a fixed order).  Calls
 * that share a workspace must be ordered on one stream.
 */
int mq_quantized_matmul_ws(const mq_bf16* x, const uint32_t* wq, const mq_bf16* scales,
                           const mq_bf16* biases, const mq_bf16* bias_vec, mq_bf16* y, int64_t M,
                           int64_t N, int64_t K, int group_size, int bits, int transpose,
                           void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * mq_quantized_matmul_ws without a workspace argument and without any
 * allocation: the split-K partial sums (and, at 2/3/5/6 bits, the codes
 * repacked one byte each) live in a device array of this library
 * (MQ_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends).  Its
 * device address is looked up (hipGetSymbolAddress) by the first call with
 * work on a device and kept once the lookup succeeds (a failed lookup returns
 * MQ_ERR_HIP and the next call retries); code that captures this entry point
 * in a HIP graph makes one eager call on the device first, so that the
 * lookup never happens during capture.  No counterpart in the reference:
 * it is for callers that cannot allocate (code under HIP graph capture,
 * serving loops that forbid hipMalloc).  Same arguments, kernels, split plan
 * and results bit for bit as mq_quantized_matmul_ws with
 * mq_quantized_matmul_workspace() bytes.  A large-M stream-K plan that needs
 * more than MQ_NOALLOC_SCRATCH_BYTES runs every tile whole instead (as
 * mq_quantized_matmul_ws does without a workspace); other shapes whose plan
 * needs more than MQ_NOALLOC_SCRATCH_BYTES (mq_quantized_matmul_workspace)
 * return MQ_ERR_INVALID before any launch.  Every call on one GPU shares its array:
 * calls that overlap on one GPU (unordered streams) race; order them on one
 * stream.  The array is used on the device of `stream` (the current device
 * for the NULL stream).
 */
#define MQ_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int mq_quantized_matmul_noalloc(const mq_bf16* x, const uint32_t* wq, const mq_bf16* scales,
                                const mq_bf16* biases, const mq_bf16* bias_vec, mq_bf16* y,
                                int64_t M, int64_t N, int64_t K, int group_size, int bits,
                                int transpose, hipStream_t stream);

/*
 * mx.gather_qmm(x, wq, scales, biases, lhs_indices, rhs_indices,
 *               transpose=True, group_size, bits, sorted_indices):
 *   y[t] = x[lhs[t]] @ dequantize(wq[rhs[t]])^T      for t < T
 * x bfloat16 [x_batches, M, K]; wq [E, N, K*bits/32]; scales/biases
 * [E, N, K/group_size]; lhs int32 [T] or NULL (identity, needs x_batches == T);
 * rhs int32 [T]; y bfloat16 [T, M, N].  sorted_indices is the caller's promise
 * that rhs is non-decreasing (models/lfm2.py:202-218 sorts when it has >= 64
 * rows), as MLX's sorted path assumes: with it and more than 64 rows, tiles are
 * cut along the experts' segments of rhs, and an rhs that is not
 * non-decreasing gives wrong rows.  Without it the result is the same for any
 * order.  A t whose lhs/rhs is out of range gets zeros.  Replaces
 * QuantizedSwitchLinear.__call__ (models/lfm2.py:176-187).
 */
int mq_gather_qmm(const mq_bf16* x, const int32_t* lhs_indices, const int32_t* rhs_indices,
                  const uint32_t* wq, const mq_bf16* scales, const mq_bf16* biases, mq_bf16* y,
                  int64_t T, int64_t M, int64_t N, int64_t K, int64_t E, int64_t x_batches,
                  int group_size, int bits, int transpose, int sorted_indices,
                  hipStream_t stream);

/*
 * mq_gather_qmm with sorted_indices = 1 for rows sorted by mq_moe_sort or
 * mq_moe_route_sort, given the segment offsets the sort wrote: expert e's
 * batches are t in [expert_offsets[e], expert_offsets[e + 1]) (int32 [E + 1],
 * device memory), batches from expert_offsets[E] on hold ids >= E (zeros).
 * The same arguments and results as mq_gather_qmm otherwise.  The sorted GEMM
 * cuts its tiles along these segments; without the offsets (mq_gather_qmm) it
 * first derives them from rhs.  With swiglu, every expert's matrix is 2N rows
 * (gate rows, then up rows: wq [E, 2N, K * bits / 32]) and y [T, M, N] =
 * mq_silu_mul of the 2N-column product, bit for bit (SwitchGLU's gate and up
 * projections and nn.silu(gate) * up, models/lfm2.py:208-214), with no
 * [T, M, 2N] intermediate; shapes it does not take return
 * MQ_ERR_UNSUPPORTED.  No counterpart in the reference: the call SwitchGLU
 * makes after _gather_sort (models/lfm2.py:176-187,204,613-618), where MLX
 * derives the segments itself.
 */
int mq_gather_qmm_segments(const mq_bf16* x, const int32_t* lhs_indices,
                           const int32_t* rhs_indices, const int32_t* expert_offsets,
                           const uint32_t* wq, const mq_bf16* scales, const mq_bf16* biases,
                           mq_bf16* y, int64_t T, int64_t M, int64_t N, int64_t K, int64_t E,
                           int64_t x_batches, int group_size, int bits, int swiglu,
                           hipStream_t stream);

/* 1 if mq_gather_qmm_segments takes these sizes (with swiglu, N is the
 * output width: every expert's matrix is 2N rows), else 0.  Without swiglu
 * every valid shape is taken (beyond the segment GEMM it runs as
 * mq_gather_qmm); with swiglu, the segment GEMM's shapes and the decode-sized
 * ones mq_gather_qmm_swiglu takes.  Host-only; no counterpart in the
 * reference. */
int mq_gather_qmm_segments_supported(int64_t T, int64_t M, int64_t N, int64_t K, int64_t E,
                                     int64_t x_batches, int group_size, int bits, int swiglu);

/*
 * SwitchGLU's gate and up projections and silu(gate) * up for gathered
 * (token, expert) pairs without the [T, M, 2N] intermediate
 * (models/lfm2.py:208-214: up_proj and gate_proj, then nn.silu(gate) * up
 * into down_proj; the two projections run as one gate|up bank): every expert's
 * matrix is 2N rows, gate rows first (wq [E, 2N, K * bits / 32], scales and
 * biases [E, 2N, K / group_size]); y bfloat16 [T, M, N] =
 * mq_silu_mul(mq_gather_qmm(x, ..., N = 2N, sorted_indices = 0)), bit for bit.
 * Arguments as mq_gather_qmm's (transpose = True).  Taken for a decode
 * step's pairs (T * M <= 64, M <= 2, rows of at most 64 lanes: where
 * mq_gather_qmm runs its per-pair GEMV); mq_gather_qmm_swiglu_supported says
 * which shapes, others return MQ_ERR_UNSUPPORTED.
 */
int mq_gather_qmm_swiglu_supported(int64_t T, int64_t M, int64_t N, int64_t K, int group_size,
                                   int bits);
int mq_gather_qmm_swiglu(const mq_bf16* x, const int32_t* lhs_indices,
                         const int32_t* rhs_indices, const uint32_t* wq, const mq_bf16* scales,
                         const mq_bf16* biases, mq_bf16* y, int64_t T, int64_t M, int64_t N,
                         int64_t K, int64_t E, int64_t x_batches, int group_size, int bits,
                         hipStream_t stream);

/* ------------------------------------------------------------------------
 * Decoder step around the quantized linears (models/qwen2.py:47-163).
 * KV pages are the reference's layout (cache.py:686-695): per layer,
 * bfloat16 [num_pages, page_size, n_kv_heads, head_dim].  A sequence's pages
 * are its row of an int32 page table [batch, pages_per_seq]; position p of
 * sequence b lives in slot page_table[b][p / page_size] * page_size +
 * p % page_size (cache.py:459-471).  positions int64 [batch] holds each
 * sequence's current token position, in device memory so that a captured
 * step replays with new values.  Out-of-range positions and page ids are
 * clamped into the cache (wrong values, never an access outside it).
 * num_pages * page_size and pages_per_seq * page_size are below 2^31.
 * ------------------------------------------------------------------------ */

/*
 * nn.RMSNorm (models/qwen2.py:140-145,187; mx.fast.rms_norm), optionally
 * fused with the residual add before it (qwen2.py:158-163):
 *   h = residual ? bf16(x + residual) : x      (h stored to residual_out)
 *   out = bf16(h * rsqrt(mean(h^2) + eps) * weight)   float32 arithmetic
 * x, residual, residual_out, out bfloat16 [rows, dim]; weight bfloat16 [dim];
 * residual and residual_out are both NULL or both set.  dim % 8 == 0, <= 8192.
 */
int mq_rms_norm(const mq_bf16* x, const mq_bf16* residual, mq_bf16* residual_out,
                const mq_bf16* weight, mq_bf16* out, int64_t rows, int64_t dim, float eps,
                hipStream_t stream);

/*
 * mx.fast.rope(traditional=False) of q and k for one token per sequence
 * (models/qwen2.py:93-108) and the paged KV append of that token
 * (cache.py:485-520, PagedBatchReservation.stage_layer):
 *   qkv bfloat16 [batch, (n_heads + 2 n_kv_heads) * head_dim] (q | k | v heads),
 *   q_out bfloat16 [batch, n_heads, head_dim] = rope(q),
 *   k_pages[slot] = rope(k), v_pages[slot] = v        (bfloat16)
 * cos/sin float32 [positions, head_dim / 2], row p = cos/sin(p * theta^(-2i/d)).
 * q_norm / k_norm (bfloat16 [head_dim] or NULL): Qwen3's per-head RMSNorm
 * before RoPE (models/qwen3.py:61-62,84-85), eps norm_eps; head_dim <= 128.
 */
int mq_rope_kv_append(const mq_bf16* qkv, const int64_t* positions, const int32_t* page_table,
                      int64_t pages_per_seq, int64_t page_size, int64_t num_pages,
                      const float* cos_table, const float* sin_table, const mq_bf16* q_norm,
                      const mq_bf16* k_norm, float norm_eps, mq_bf16* q_out, mq_bf16* k_pages,
                      mq_bf16* v_pages, int64_t batch, int n_heads, int n_kv_heads, int head_dim,
                      hipStream_t stream);

/*
 * Workspace, in bytes, for mq_paged_decode_attention (0 = unsupported shape).
 * Positions are split over blocks; each split leaves float32 partials.  No
 * counterpart in the reference (MLX allocates temporaries internally).
 */
size_t mq_paged_decode_attention_workspace(int64_t batch, int n_heads, int n_kv_heads,
                                           int head_dim, int64_t pages_per_seq,
                                           int64_t page_size);

/*
 * Attention of one query token per sequence over its cached positions
 * 0..positions[b] (causal, grouped-query: query head h reads KV head
 * h / (n_heads / n_kv_heads)).  Replaces PagedLayerAttentionContext
 * .append_and_attend's gather of the pages into dense rows plus
 * mx.fast.scaled_dot_product_attention for a decode step
 * (attention.py:206-298).  q bfloat16 [batch, n_heads, head_dim];
 * out bfloat16 [batch, n_heads * head_dim]; float32 softmax and accumulation.
 * head_dim 64 or 128, 1-8 query heads per KV head.
 */
int mq_paged_decode_attention(const mq_bf16* q, const mq_bf16* k_pages, const mq_bf16* v_pages,
                              const int32_t* page_table, int64_t pages_per_seq, int64_t page_size,
                              int64_t num_pages, const int64_t* positions, int64_t batch,
                              int n_heads, int n_kv_heads, int head_dim, float scale,
                              void* workspace, size_t workspace_bytes, mq_bf16* out,
                              hipStream_t stream);

/*
 * Causal attention of a prefill chunk over the paged cache: query token j of
 * row b sits at position starts[b] + min(j, lens[b] - 1) (tokens past
 * lens[b] are padding that repeats the row's last position) and attends to
 * the row's cached positions 0..that position (grouped-query: query head h
 * reads KV head h / (n_heads / n_kv_heads)); the chunk's own k and v must
 * already be in the pages.  Replaces PagedLayerAttentionContext
 * .append_and_attend's dense gather of the pages, _dense_causal_mask and
 * mx.fast.scaled_dot_product_attention for a prefill chunk
 * (attention.py:215-261,404-425).  q bfloat16 [batch, tokens, n_heads,
 * head_dim] (roped); starts, lens int64 [batch]; page_table int32 [batch,
 * pages_per_seq] (the batch's rows); out bfloat16 [batch, tokens, n_heads,
 * head_dim].  float32 scores, softmax and accumulation, the probabilities
 * rounded to bfloat16 for the products with v.  head_dim 128; the pages of
 * one layer under 2 GiB.
 */
/* 1 if mq_paged_prefill_attention takes these sizes, else 0.  Host-only; no
 * counterpart in the reference. */
int mq_paged_prefill_attention_supported(int n_heads, int n_kv_heads, int head_dim,
                                         int64_t num_pages, int64_t page_size);

int mq_paged_prefill_attention(const mq_bf16* q, const mq_bf16* k_pages, const mq_bf16* v_pages,
                               const int32_t* page_table, int64_t pages_per_seq,
                               int64_t page_size, int64_t num_pages, const int64_t* starts,
                               const int64_t* lens, int64_t batch, int64_t tokens, int n_heads,
                               int n_kv_heads, int head_dim, float scale, mq_bf16* out,
                               hipStream_t stream);

/*
 * One decode step of a layer's attention after its QKV projection:
 * mq_rope_kv_append followed by mq_paged_decode_attention (same arguments and
 * results, bit for bit) with the RoPE (and Qwen3's q/k norms) and the append
 * of k and v done inside the attention's split kernel -- two launches instead
 * of three.  Replaces the part of Qwen2Attention.__call__ after the
 * projections (models/qwen2.py:93-113): rope +
 * PagedLayerAttentionContext.append_and_attend (attention.py:206-298).  The
 * workspace is mq_paged_decode_attention_workspace() bytes.
 */
int mq_decode_attention_step(const mq_bf16* qkv, const int64_t* positions,
                             const int32_t* page_table, int64_t pages_per_seq, int64_t page_size,
                             int64_t num_pages, const float* cos_table, const float* sin_table,
                             const mq_bf16* q_norm, const mq_bf16* k_norm, float norm_eps,
                             mq_bf16* k_pages, mq_bf16* v_pages, int64_t batch, int n_heads,
                             int n_kv_heads, int head_dim, float scale, void* workspace,
                             size_t workspace_bytes, mq_bf16* out, hipStream_t stream);

/*
 * silu(gate) * up of the MLP (models/qwen2.py:43-44,132-133) on the fused
 * gate|up projection: gate_up bfloat16 [rows, 2 * inter], out bfloat16
 * [rows, inter] = bf16(bf16(gate * sigmoid(gate)) * up).  inter % 8 == 0.
 */
int mq_silu_mul(const mq_bf16* gate_up, mq_bf16* out, int64_t rows, int64_t inter,
                hipStream_t stream);

/*
 * The MLP's gate|up projection and silu(gate) * up without the [M, 2N]
 * intermediate (models/qwen2.py:132-133: down(silu(gate(x)) * up(x)) up to
 * the down projection): wq [2N, K * bits / 32] with the gate rows first (as
 * the fused gate|up matrix of mq_quantized_matmul), y bfloat16 [M, N] =
 * mq_silu_mul(mq_quantized_matmul_ws(x, wq, ...)), bit for bit.  Taken for
 * decode shapes: M <= 2 on large matrices (2*N*K >= 2^25, K rows of at most 64
 * lanes: the dot2 GEMV with a SwiGLU epilogue, no workspace), and the skinny
 * GEMM's split-K plans (e.g. M = 32: its fixed-order reduce applies the
 * SwiGLU; needs mq_quantized_matmul_swiglu_workspace bytes, which is what
 * mq_quantized_matmul_workspace gives the unfused product); and for prefill
 * shapes the large-M GEMM runs every tile whole (SiLU * up in its epilogue,
 * no workspace; bit for bit mq_quantized_matmul_ws without a workspace,
 * followed by mq_silu_mul).
 * mq_quantized_matmul_swiglu_supported says whether a shape is taken; others
 * return MQ_ERR_UNSUPPORTED.  mq_quantized_matmul_swiglu is the _ws form
 * without a workspace.
 */
int mq_quantized_matmul_swiglu_supported(int64_t M, int64_t N, int64_t K, int group_size,
                                         int bits);
size_t mq_quantized_matmul_swiglu_workspace(int64_t M, int64_t N, int64_t K, int group_size,
                                            int bits);
int mq_quantized_matmul_swiglu_ws(const mq_bf16* x, const uint32_t* wq, const mq_bf16* scales,
                                  const mq_bf16* biases, mq_bf16* y, int64_t M, int64_t N,
                                  int64_t K, int group_size, int bits, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream);
int mq_quantized_matmul_swiglu(const mq_bf16* x, const uint32_t* wq, const mq_bf16* scales,
                               const mq_bf16* biases, mq_bf16* y, int64_t M, int64_t N, int64_t K,
                               int group_size, int bits, hipStream_t stream);

/*
 * A quantized linear followed by the residual add and the RMSNorm that read
 * its output (models/qwen2.py:162-163 hidden = x + attn_out ->
 * post_attention_layernorm; :164 hidden + mlp_out -> the next layer's
 * input_layernorm or the final norm :199):
 *   y = x @ dequantize(wq)^T (+ bias)        bfloat16, as mq_quantized_matmul_ws
 *   h = bf16(y + residual)                   -> residual_out
 *   out = bf16(h * rsqrt(mean(h^2) + eps) * norm_weight)
 * equal bit for bit to mq_quantized_matmul_ws (with its workspace) followed by
 * mq_rms_norm(y, residual, ...).  Taken for the skinny GEMM's split-K plans
 * with N <= 8192 (e.g. the o and down projections at decode batch 32: the
 * split-K reduce does the add and the norm, one launch fewer);
 * mq_quantized_matmul_add_rms_norm_supported says which.  x [M, K],
 * residual, residual_out, out [M, N], norm_weight [N], all bfloat16.
 */
int mq_quantized_matmul_add_rms_norm_supported(int64_t M, int64_t N, int64_t K, int group_size,
                                               int bits);
size_t mq_quantized_matmul_add_rms_norm_workspace(int64_t M, int64_t N, int64_t K,
                                                  int group_size, int bits);
int mq_quantized_matmul_add_rms_norm(const mq_bf16* x, const uint32_t* wq, const mq_bf16* scales,
                                     const mq_bf16* biases, const mq_bf16* bias_vec,
                                     const mq_bf16* residual, mq_bf16* residual_out,
                                     const mq_bf16* norm_weight, float eps, mq_bf16* out,
                                     int64_t M, int64_t N, int64_t K, int group_size, int bits,
                                     void* workspace, size_t workspace_bytes,
                                     hipStream_t stream);

/*
 * mq_rms_norm of one row followed by the quantized linear that reads it, in
 * one kernel (the decoder's norm -> linear pairs, models/qwen2.py:157
 * input_layernorm -> q/k/v, :162-163 hidden = x + attn_out,
 * post_attention_layernorm -> gate|up, :199 final norm -> lm_head :227):
 *   h = residual ? bf16(a + residual) : a          (h -> residual_out)
 *   x = bf16(h * rsqrt(mean(h^2) + eps) * norm_weight)   as mq_rms_norm, bit for bit
 *   y = x @ dequantize(wq)^T (+ bias)                   as the dot2 GEMV
 *   or, with swiglu, y [1, N] = silu(gate) * up of a [2N, K] gate|up matrix
 *   (as mq_quantized_matmul_swiglu).
 * a, residual, residual_out, norm_weight bfloat16 [K]; M must be 1 and
 * K <= 8192; residual_out may not overlap a or residual (every block reads
 * them while the first writes it).  mq_rms_norm_quantized_matmul_supported
 * says whether a shape is taken; others return MQ_ERR_UNSUPPORTED.
 */
int mq_rms_norm_quantized_matmul_supported(int64_t M, int64_t N, int64_t K, int group_size,
                                           int bits, int swiglu);
int mq_rms_norm_quantized_matmul(const mq_bf16* a, const mq_bf16* residual, mq_bf16* residual_out,
                                 const mq_bf16* norm_weight, float eps, const uint32_t* wq,
                                 const mq_bf16* scales, const mq_bf16* biases,
                                 const mq_bf16* bias_vec, mq_bf16* y, int64_t M, int64_t N,
                                 int64_t K, int group_size, int bits, int swiglu,
                                 hipStream_t stream);

/* ------------------------------------------------------------------------
 * Mixture-of-experts routing around mq_gather_qmm (models/lfm2.py:348-375,
 * SwitchGLU lfm2.py:193-218 with _gather_sort/_scatter_unsort :613-622).
 * ------------------------------------------------------------------------ */

/*
 * Router of Lfm2MoE.__call__ (models/lfm2.py:365-373) after the gate linear:
 *   gates = softmax(float32(logits)) (+ expert_bias, float32 [E], or NULL)
 *   indices int32 [tokens, top_k] = the top_k gates' experts (argpartition;
 *     here in descending gate order, ties to the lower id),
 *   scores bfloat16 [tokens, top_k] = those gates, divided by
 *     (their sum + 1e-20) when norm_topk_prob.
 * logits bfloat16 [tokens, num_experts]; num_experts <= 512, top_k <= 64.
 */
int mq_moe_route(const mq_bf16* logits, const float* expert_bias, int64_t tokens,
                 int num_experts, int top_k, int norm_topk_prob, int32_t* indices,
                 mq_bf16* scores, hipStream_t stream);

/*
 * _gather_sort (models/lfm2.py:613-618) as a stable counting sort of the flat
 * expert ids [n] (n = tokens * top_k): sorted_ids[p] = ids[order[p]],
 * inverse[order[p]] = p, and rows[p] = order[p] / top_k (the x row that
 * mq_gather_qmm takes as lhs index; rows may be NULL).  Ids outside
 * [0, num_experts) sort last, unchanged.  expert_offsets (int32
 * [num_experts + 1], or NULL) receives where each expert's run of sorted_ids
 * starts (the last entry counts the ids inside [0, num_experts)), for
 * mq_gather_qmm_segments.  int32 throughout; one block.
 */
int mq_moe_sort(const int32_t* expert_ids, int64_t n, int top_k, int num_experts,
                int32_t* sorted_ids, int32_t* order, int32_t* inverse, int32_t* rows,
                int32_t* expert_offsets, hipStream_t stream);

/*
 * _scatter_unsort (models/lfm2.py:621-622) and the score-weighted sum over the
 * top_k experts (lfm2.py:375):
 *   out[t, :] = bf16( sum_j bf16(y[r(t, j), :] * scores[t, j]) ),  float32 sum,
 * r(t, j) = inverse[t * top_k + j] (rows of y in expert order), or
 * t * top_k + j when inverse is NULL.  y bfloat16 [tokens * top_k, hidden],
 * out bfloat16 [tokens, hidden], hidden % 8 == 0.
 */
int mq_moe_combine(const mq_bf16* y, const int32_t* inverse, const mq_bf16* scores, mq_bf16* out,
                   int64_t tokens, int top_k, int64_t hidden, hipStream_t stream);

/*
 * mq_moe_route then mq_moe_sort of the routed indices [tokens, top_k], with
 * the same outputs bit for bit (the router of models/lfm2.py:365-373 and
 * _gather_sort :613-618, which the reference runs back to back).  Up to 64
 * tokens run as one block and one launch; more run as the two kernels.
 */
int mq_moe_route_sort(const mq_bf16* logits, const float* expert_bias, int64_t tokens,
                      int num_experts, int top_k, int norm_topk_prob, int32_t* indices,
                      mq_bf16* scores, int32_t* sorted_ids, int32_t* order, int32_t* inverse,
                      int32_t* rows, int32_t* expert_offsets, hipStream_t stream);

/*
 * Greedy decoding's next token: out int64 [rows] = the first index of each
 * row's largest value, x bfloat16 [rows, cols] (cols % 8 == 0, cols <= 2^28,
 * x 16-byte aligned; -0 equals +0, NaN counts as the largest, as torch.argmax returns
 * the first NaN).  Replaces mx.argmax over the last logits of each row, as
 * the reference's executor takes the next tokens (executor.py:406-414).
 */
int mq_argmax_rows(const mq_bf16* x, int64_t rows, int64_t cols, int64_t* out,
                   hipStream_t stream);

/*
 * mq_moe_combine, then the residual add and the RMSNorm that follow the MoE
 * block (models/lfm2.py:409 hidden + feed_forward(...), then the next layer's
 * operator_norm :404 or the final embedding_norm :436), one kernel per token:
 *   h = bf16(combine(y, inverse, scores) + residual)      -> residual_out
 *   out = bf16(h * rsqrt(mean(h^2) + eps) * weight)
 * Bit-identical to mq_moe_combine followed by mq_rms_norm(combined, residual,
 * ...).  hidden % 8 == 0, <= 8192; residual_out may not alias residual.
 */
int mq_moe_combine_rms_norm(const mq_bf16* y, const int32_t* inverse, const mq_bf16* scores,
                            const mq_bf16* residual, mq_bf16* residual_out,
                            const mq_bf16* weight, mq_bf16* out, int64_t tokens, int top_k,
                            int64_t hidden, float eps, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MQ_H */
