/*
 * mq_measure.h -- measurement helper of libmi355q (no counterpart in the
 * reference: it exists so that a benchmark can time the hardware floor the
 * quantized GEMV is compared with).
 */
#ifndef MQ_MEASURE_H
#define MQ_MEASURE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Read `bytes` bytes at device address src once, in the decode GEMV's load
 * pattern (16-byte non-temporal buffer loads, 64 consecutive chunks per wave
 * instruction), and write nothing unless the XOR of every word is 0x9e3779b9
 * (then that value to sink[0]): one launch whose time is the read-only HBM
 * floor for a kernel streaming the same bytes.  src 16-byte aligned, bytes a
 * multiple of 16 and below 2^32.  Returns MQ_OK (0), MQ_ERR_INVALID (-1) or
 * MQ_ERR_HIP (-3); the message is mq_last_error()'s.
 */
int mq_hbm_read(const void* src, size_t bytes, uint32_t* sink, hipStream_t stream);

/*
 * The one-row 4-bit GEMV of mq_quantized_matmul (M = 1, group size 64, K 3584
 * or 4096, N large enough that it runs 16 lanes per row), y = x . W^T, with a
 * per-wave timeline: trace[4 * w + 0..2] are the 100 MHz constant clock
 * (s_memrealtime) at wave w's entry, after its block's prologue barrier (x
 * staged) and after its store; trace[4 * w + 3] is XCC_ID << 32 | HW_ID (the
 * CU it ran on).  Waves are numbered block by block, four per block of 16
 * rows.  trace_words >= 4 * waves.  y equals mq_quantized_matmul's bit for
 * bit.  For measurement only (the phase times of the decode GEMV).
 */
int mq_qmv_trace(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                 const uint16_t* biases, uint16_t* y, int64_t N, int64_t K, uint64_t* trace,
                 size_t trace_words, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MQ_MEASURE_H */
