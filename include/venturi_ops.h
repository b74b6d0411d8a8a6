/*
 * libventuri_ops.so: C ABI of the gfx950 (MI355X) quantized-linear library.
 *
 * Conventions shared with the reference's operator ABI
 * (/root/reference/src/venturi/ops/csrc/ops_api.h):
 *   - return 0 on success, -1 on invalid input or launch failure with a
 *     per-thread message from venturi_blocks_error(); *_bytes return 0 on error;
 *   - dtype codes 0 = fp16, 1 = bf16, 2 = fp32;
 *   - `padded` must equal ceil(k/128)*128; Q8 codes are int8 [n][padded],
 *     Q8 scales fp16 [n][padded/32];
 *   - `stream` is a hipStream_t (torch.cuda.current_stream().cuda_stream);
 *   - no entry point allocates device memory or synchronises; all buffers are
 *     caller-owned. Launches are graph-capturable.
 * Alignment: Q8 codes and A8 workspaces 16 bytes; fp16/bf16 operands 2 bytes
 * (the reference accepts unaligned Q8 codes; this library requires 16).
 */
#ifndef VENTURI_OPS_H
#define VENTURI_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Identity. ABI 18 as ops_api.h:6 (blocks.cu:650-652); the arch tag is 950. */
int venturi_blocks_abi(void);
int venturi_blocks_arch(void);
const char* venturi_blocks_error(void);

/* Q8 A16 projection out[t][n] = sum_k x[t][k] * code[n][k] * scale[n][k/32],
 * in the reference's canonical fp32 order (bytes identical to q8_head).
 * Replaces ops_api.h:62-63 / blocks.cu:935-948. */
int venturi_q8_head_run(const void* x, const int8_t* codes, const void* scales, void* out, int tokens,
                        int vocab, int k, int padded, int dtype, void* stream);

/* Q8 row lookup out[i][c] = code[ids[i]][c] * scale; ids outside [0, vocab)
 * give zero rows. Replaces ops_api.h:56-57 / blocks.cu:918-934. */
int venturi_q8_embedding_run(const int8_t* codes, const void* scales, const int64_t* ids, void* out,
                             int tokens, int vocab, int k, int padded, int dtype, void* stream);

/* A8 workspace size: tokens*ceil(k/32)*36*passes bytes (passes 1 or 2).
 * Replaces ops_api.h:53 / q8_dp4a.cuh:7-13, 90-92. */
uint64_t venturi_q8_dp4a_bytes(int tokens, int k, int passes);

/* fp16 x -> int8 codes [pass][t][group][32] + fp32 scales [pass][t][group].
 * Replaces ops_api.h:54 / q8_dp4a.cuh:93-101. */
int venturi_q8_dp4a_quantize(const void* x, void* workspace, uint64_t available, int tokens, int k, int passes,
                             void* stream);

/* W8A8 projection of a quantized workspace, fp16 out, reference order.
 * Replaces ops_api.h:55 / q8_dp4a.cuh:102-109. */
int venturi_q8_dp4a_run(const void* workspace, uint64_t available, const int8_t* codes, const void* scales,
                        void* out, int tokens, int n, int k, int padded, int passes, void* stream);

/* RMSNorm out = (x * 1/sqrt(mean(x^2) + eps)) * w, fp32 w.
 * Replaces ops_api.h:93-94 / blocks.cu:727-740. */
int venturi_rms_run(const void* x, const float* w, void* out, int tokens, int features, int dtype, float epsilon,
                    void* stream);

/* RMSNorm -> fp16 -> two-pass A8 workspace; `chunk` in {8,32,128} is accepted
 * for compatibility. Replaces ops_api.h:91-92 / q8_rms_producer.cuh:67-84. */
int venturi_rms_q8_quantize(const void* x, const float* w, void* workspace, uint64_t available, int tokens, int k,
                            float epsilon, int chunk, void* intermediate, void* stream);

/* Extension (no reference counterpart: its fused producer is two-pass only):
 * the same producer with passes in {1, 2}. */
int venturi_rms_q8_quantize_passes(const void* x, const float* w, void* workspace, uint64_t available, int tokens,
                                   int k, float epsilon, int passes, void* intermediate, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VENTURI_OPS_H */
