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
 *   - no entry point allocates device memory or synchronises (except the first
 *     call of the hipBLASLt-backed entry points, venturi_dense_run and the
 *     *_dense_run projections, per device and shape); all buffers are
 *     caller-owned. Launches are graph-capturable.
 * Alignment: venturi_q8_head_run and venturi_q8_embedding_run take Q8 codes
 * at any address, as the reference does (a row-offset view of a plane); the
 * matrix-core Q8 entry points, the A8 projections and their workspaces need
 * 16-byte codes and workspaces; fp16/bf16 operands 2 bytes.
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

/* Extension (no counterpart in the reference): the same W8A8 projection on
 * int-exact fp16 matrix cores, with the 32-column group dots exact (as the
 * reference's int32 accumulators) and the scaled group terms summed in
 * natural order, so outputs match the reference to fp32 association. Same
 * arguments and workspace as venturi_q8_dp4a_run. */
int venturi_q8_a8_gemm_run(const void* workspace, uint64_t available, const int8_t* codes, const void* scales,
                           void* out, int tokens, int n, int k, int padded, int passes, void* stream);

/* Extension (no counterpart in the reference): the same W8A8 projection at
 * 1..32 tokens on int8 matrix cores (v_mfma_i32_16x16x32_i8: one exact int32
 * group dot per 32-column group) over the tiled Q8 planes that
 * venturi_q8_tiled_run reads (codes [block][chunk][lane][16 B], scales
 * [block][chunk][row][2]); the scaled group terms summed in natural order, so
 * outputs match the reference to fp32 association. Same workspace as
 * venturi_q8_dp4a_run; workspace and planes 16-byte aligned. Shapes whose
 * launch splits K over two workgroups take `slots`: at least
 * venturi_q8_a8_tiled_workspace_bytes bytes, 8-byte aligned, armed once with
 * venturi_q8_tiled_workspace_init and left idle by every run (calls sharing
 * one slot buffer run on one stream); NULL / 0 for the other shapes. */
int venturi_q8_a8_tiled_run(const void* workspace, uint64_t available, const void* codes, const void* scales,
                            void* out, int tokens, int n, int k, int padded, int passes, void* slots,
                            uint64_t slot_bytes, void* stream);

/* Extension (no counterpart in the reference): venturi_q8_dp4a_quantize
 * (q8_dp4a.cuh:15-45) of fp16 x [tokens][k] into the workspace followed by
 * venturi_q8_a8_tiled_run, as one launch when tokens <= 16, k % 8 == 0, x is
 * 16-byte aligned and the quantized activations fit 64 KB of LDS (each
 * workgroup quantizes them itself), else as the two launches. Either way the
 * workspace ends holding the quantizer's bytes and out the bytes of the two
 * calls. Slots as for venturi_q8_a8_tiled_run. */
int venturi_q8_a8_tiled_linear_run(const void* x, void* workspace, uint64_t available, const void* codes,
                                   const void* scales, void* out, int tokens, int n, int k, int padded, int passes,
                                   void* slots, uint64_t slot_bytes, void* stream);

/* Extension (no counterpart in the reference): bytes of the exchange slots the
 * two A8 entry points above need at this shape; 0 when its launch does not
 * split K, and 0 with a message for invalid geometry. */
uint64_t venturi_q8_a8_tiled_workspace_bytes(int tokens, int n, int k, int passes);

/* One matrix of a fused projection: resident Q8 planes, its fp16 output
 * [tokens][stride] (rows n, stride >= n). 32 bytes, as ops_api.h:8-9. */
typedef struct VQFOutput {
    const int8_t* codes;
    const void* scales;
    void* out;
    int n, stride;
} VQFOutput;

/* Two or three Q8 matrices of one K against one A8 workspace, each output
 * written with its own row stride; bytes equal venturi_q8_dp4a_run per matrix
 * (reference order). One launch below 64 tokens. Replaces ops_api.h:61 /
 * q8_fused.cuh:186-205. */
int venturi_q8_fused_run(const void* workspace, uint64_t available, const VQFOutput* outputs, int count, int tokens,
                         int k, int padded, int passes, void* stream);

/* SwiGLU of gate and up (fp16 [tokens][k]) rounded to fp16, then two-pass A8
 * into `workspace` (venturi_q8_dp4a_bytes(tokens, k, 2)); optional
 * `intermediate_debug` receives the rounded SwiGLU values; threads 128 or
 * 256. Bytes equal venturi_swiglu_run followed by venturi_q8_dp4a_quantize.
 * Replaces ops_api.h:99-100 / q8_producer.cuh:60-82. */
int venturi_swiglu_q8_quantize(const void* gate, const void* up, void* workspace, uint64_t available, int tokens,
                               int k, int threads, void* intermediate_debug, void* stream);

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

/* Extension (the reference packs Q8 on the CPU only, weights.py:398-439):
 * device Q8 packing of a dense fp16/bf16/fp32 [n][k] source with the
 * arithmetic of Q8RowSplitWeight.from_dense; codes/scales bytes identical. */
int venturi_q8_pack_run(const void* source, int8_t* codes, void* scales, int n, int k, int padded, int dtype,
                        void* stream);

/* Extension: Q8 A16 projection on fp16 matrix cores (same arguments as
 * venturi_q8_head_run; fp16 activations, k % 8 == 0, tokens <= 16). Per-group
 * fp32 scaling of exact group dots; agrees with the canonical order to fp32
 * association, not bit-for-bit. */
int venturi_q8_gemm_run(const void* x, const int8_t* codes, const void* scales, void* out, int tokens, int n, int k,
                        int padded, int dtype, void* stream);

/* Extension: the same projection for many tokens (prefill) on fp16 matrix
 * cores over the row-major planes: LDS-staged 256-token x 128-row tiles,
 * codes converted to fp16 once per tile, one fp32 scale FMA per 32-column
 * group. fp16 activations, k % 8 == 0, 16-byte aligned x; any token count. */
int venturi_q8_prefill_run(const void* x, const int8_t* codes, const void* scales, void* out, int tokens, int n, int k,
                           int padded, int dtype, void* stream);

/* Extension: workspace of the tiled projections below for (tokens, n, swiglu):
 * the exchange slots of launches that split K over two workgroups, or 0 when
 * no launch for (tokens, n) splits. The size does not depend on K: at one
 * token, 4097-6144 rows reserve slots that only rows of more than 8064
 * columns use. 0 with a message on invalid arguments (tokens outside 1..32,
 * n <= 0, odd n with swiglu). */
size_t venturi_q8_tiled_workspace_bytes(int tokens, int n, int swiglu);

/* Extension: puts a workspace of the tiled projections in its idle state (every
 * 64-bit word 0x7f8000017f800001) with a fill kernel on `stream`. Call it once
 * after allocating; every projection call leaves the workspace idle again.
 * Calls that share one workspace must be ordered (one stream). */
int venturi_q8_tiled_workspace_init(void* workspace, size_t bytes, void* stream);

/* Extension: the same projection over tiled planes: row blocks of 16 rows x
 * 64-column chunks, 1 KB each, stored [block][chunk][lane 16q+m][16 bytes]
 * (row m's codes of columns 64c+8q..+8, then 64c+32+8q..+8), scales
 * [block][chunk][m][2] fp16; each wave then streams contiguous 1 KB blocks.
 * fp16 activations, k % 8 == 0, tokens <= 32. `workspace` (8-byte aligned,
 * initialised, at least venturi_q8_tiled_workspace_bytes) may be NULL when
 * that size is 0. */
int venturi_q8_tiled_run(const void* x, const void* codes, const void* scales, void* out, int tokens, int n, int k,
                         int padded, int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* No counterpart in the reference. For callers that cannot allocate (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc):
 * venturi_q8_tiled_run without the workspace arguments. The exchange slots of
 * launches that split K live in a static 1 MiB device array held per GPU until
 * the process ends (every split shape fits; larger needs are rejected with a
 * message). The first call on a device fills the slots on `stream` and must
 * run outside graph capture; every call leaves them idle. All calls on one GPU
 * share the array, so calls that overlap in time on one GPU race. Allocates
 * nothing. */
int venturi_q8_tiled_run_noalloc(const void* x, const void* codes, const void* scales, void* out, int tokens, int n,
                                 int k, int padded, int dtype, void* stream);

/* Extension (no counterpart in the reference; the native runtime runs the
 * gate+up projection and then SwiGLU, blocks.cu:56-86): the fused gate+up
 * projection over paired tiled planes (16-row block b holds gate rows
 * 8b..8b+7 then up rows n/2+8b..n/2+8b+7, built by vocabulary.tile_q8 with
 * paired=True), writing out [tokens][n/2] = fp16(swiglu(fp16(gate), fp16(up))),
 * the bytes of venturi_q8_tiled_run followed by venturi_silu_mul_run. fp16
 * activations, k % 8 == 0, n even, tokens <= 32; workspace as for
 * venturi_q8_tiled_run, sized with swiglu = 1. */
int venturi_q8_tiled_swiglu_run(const void* x, const void* codes, const void* scales, void* out, int tokens, int n,
                                int k, int padded, int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* ---- Q4 (q4_g64_fp16): codes uint8 [n][padded/2] (column 2j in the low
 * nibble of byte j, two's complement), scales fp16 [n][padded/64]. ---- */

/* Extension (the reference encodes on the CPU only, flash_next_q4.py:26-52):
 * quantize_q4_rtn of a dense fp16/bf16/fp32 [n][k] source on the device;
 * codes/scales bytes identical to the CPU encoder. */
int venturi_q4_pack_run(const void* source, void* codes, void* scales, int n, int k, int padded, int dtype,
                        void* stream);

/* Expert operator ABI 1 (flash_next_q4.cu:36-54). These two return a HIP error
 * code (0 = success, hipErrorInvalidValue on bad arguments), as the reference
 * returns a CUDA error code; padded >= k with padded % 128 == 0. */
int venturi_q4_abi(void); /* returns 1 */
/* fp16 matrix fp16(q * scale) [rows][cols]. Replaces flash_next_q4.cu:37-46. */
int venturi_q4_decode(const void* codes, const void* scales, void* out, int rows, int cols, int padded,
                      void* stream);
/* Expert GEMV, 1..64 fp16 tokens, fp16(q*scale) weights in the lane-strided
 * fmaf order; bytes identical. Replaces flash_next_q4.cu:47-54. */
int venturi_q4_linear(const void* x, const void* codes, const void* scales, void* out, int tokens, int rows,
                      int cols, int padded, void* stream);

/* Research fused Q4 GEMV (FP32 scaled integer products), fp16 only; bytes
 * identical to q4_fused_run_kernel. Replaces ops_api.h:49 / blocks.cu:1067-1076. */
int venturi_q4_fused_run(const void* x, const void* codes, const void* scales, void* out, int t, int rows, int k,
                         int padded, int dtype, void* stream);

/* Row-codec decode of rows [row, row+rows) into out [rows][k] fp16 (ld = k),
 * bits 4, 5 or 6: codes [n][padded/2] low nibbles, high plane
 * [n][padded*(bits-4)/8] (LSB-first stream of the upper bits; unused for 4),
 * scales [n][padded/64]; w = fp16(q*scale). Replaces ops_api.h:98 /
 * blocks.cu:1077-1086, weight_dequant.cuh:16-59. */
int venturi_row_dequant_rows(const void* codes, const void* high, const void* scales, void* out, int row, int rows,
                             int k, int padded, int bits, void* stream);

/* The same decode of `count` rows named by int64 `ids` (each must be a row of
 * the planes) into out [count][k]. Replaces ops_api.h / blocks.cu:1088-1096,
 * weight_dequant.cuh:61-67. */
int venturi_row_dequant_indexed(const void* codes, const void* high, const void* scales, const int64_t* ids,
                                void* out, int count, int k, int padded, int bits, void* stream);

/* W5A16 operator ABI 1 (flash_next_q5.cu:40-64): returns a HIP error code
 * (hipErrorInvalidValue on bad arguments) like the Q4 expert ABI. */
int venturi_q5_abi(void); /* returns 1 */
/* fp16 decode of a q5_g64_fp16 matrix [rows][cols]. Replaces
 * flash_next_q5.cu:42-52. */
int venturi_q5_decode(const void* codes, const void* high, const void* scales, void* out, int rows, int cols,
                      int padded, void* stream);
/* W5A16 GEMV, 1..64 fp16 tokens, fp16(q*scale) weights in the lane-strided
 * fmaf order; bytes identical. Replaces flash_next_q5.cu:53-64. */
int venturi_q5_linear(const void* x, const void* codes, const void* high, const void* scales, void* out, int tokens,
                      int rows, int cols, int padded, void* stream);

/* Plugin ABI 2 (q4_linear.cu:60-88): its own thread-local error text. */
int venturi_ada_abi(void); /* returns 2 */
const char* venturi_ada_error(void);
/* Admission: returns route 0 (requested -1 auto or 0 generic) or -1. Device
 * must be gfx950. Replaces q4_linear.cu:62-75. */
int venturi_q4_prepare(int n, int k, int tokens, int dtype, int requested);
/* FP32-weight SIMT order, fp16/bf16 (dtype 0/1), padded_k == ceil(k/128)*128;
 * bytes identical. Replaces q4_linear.cu:76-88. */
int venturi_q4_run(const void* x, const void* codes, const void* scales, void* out, int n, int k, int padded_k,
                   int tokens, int dtype, int route, void* stream);

/* Extension: the W4A16 contract GEMM (fp16(q*scale) weights, fp32 accumulation
 * on fp16 matrix cores), fp16 activations, k % 8 == 0, x 16-byte aligned, any
 * token count. Stands where the reference dequantizes to an fp16 shadow and
 * calls cuBLAS (row_codec_dispatch.cuh:41-48, qwen_runtime.cuh:348-364). */
int venturi_q4_gemm_run(const void* x, const void* codes, const void* scales, void* out, int tokens, int n, int k,
                        int padded, int dtype, void* stream);

/* Extension: the same contract GEMM at decode token counts (1..31) over the
 * tiled decode copy of the planes (q4.tile_q4: codes [ceil(n/16)][padded/128]
 * [64 lanes][16 bytes] of biased, reordered nibbles, scales
 * [ceil(n/16)][padded/128][16][2] fp16, rows past n zero); fp16 activations,
 * k % 8 == 0, x and codes 16-byte aligned, scales 4-byte aligned. Shapes that
 * split K over two workgroups (venturi_q4_tiled_workspace_bytes > 0) need a
 * slot buffer of that size, put idle once by venturi_q4_tiled_workspace_init;
 * calls sharing it run on one stream. Unsplit shapes give the bits of
 * venturi_q4_gemm_run on the row-major planes. No counterpart in the reference
 * (which streams its Q4 shadow through cuBLAS); for callers that decode from a
 * resident tiled copy. */
uint64_t venturi_q4_tiled_workspace_bytes(int tokens, int n, int k);
int venturi_q4_tiled_workspace_init(void* workspace, uint64_t bytes, void* stream);
int venturi_q4_tiled_run(const void* x, const void* codes, const void* scales, void* out, int tokens, int n, int k,
                         int padded, int dtype, void* workspace, uint64_t workspace_bytes, void* stream);

/* Extension: venturi_q4_tiled_run for 4-, 5- and 6-bit row codecs: bits 4 reads
 * the copy described above; bits 5/6 read q5.tile_row_codec's copy (codes tiled
 * as for Q4 with the nibbles unbiased; high plane [ceil(n/16)][padded/128][64
 * lanes][bits-4 32-bit registers], each column's upper bits with the sign bit
 * flipped, the pair (c+2m, c+2m+1) of the lane's word j at bits (bits-4)*jj +
 * (0, 8, 4, 12)[m] and 16 above in register j / (4/(bits-4)), jj = j mod
 * 4/(bits-4); scales as for Q4; high 4-byte aligned). Same
 * slot buffer rule; unsplit shapes give the bits of venturi_row_gemm_run on the
 * row-major planes. No counterpart in the reference; for callers that decode
 * q5/q6 rows from a resident tiled copy. */
int venturi_row_tiled_run(const void* x, const void* codes, const void* high, const void* scales, void* out,
                          int tokens, int n, int k, int padded, int bits, int dtype, void* workspace,
                          uint64_t workspace_bytes, void* stream);

/* Extension: the same contract GEMM for 4-, 5- and 6-bit row codecs (bits
 * 4/5/6; `high` = the q5/q6 high plane [n][padded*(bits-4)/8], 16-byte
 * aligned, unused for 4 bits). Stands where the reference dequantizes q4/q5/q6
 * rows to an fp16 shadow chunk and calls a dense GEMM
 * (row_codec_dispatch.cuh:41-46, weight_dequant.cuh:1-9). */
int venturi_row_gemm_run(const void* x, const void* codes, const void* high, const void* scales, void* out, int tokens,
                         int n, int k, int padded, int bits, int dtype, void* stream);

/* The reference's ChunkedDense W*A16 projection for q4/q5/q6_g64 (admitted by
 * row_codec_dispatch.cuh:41-48, run by row_dense_project,
 * qwen_runtime.cuh:348-364): chunks of rows are decoded to fp16(q*scale) into
 * the workspace and multiplied by one hipBLASLt GEMM each (fp16 operands, fp32
 * accumulation), written straight into out's columns. fp16 activations only;
 * k % 8 == 0, n % 8 == 0; x and out 16-byte aligned, workspace 256-byte
 * aligned. venturi_row_dense_workspace_bytes gives the workspace of the
 * preferred chunking (0 on invalid geometry); a smaller one (at least 32 MiB
 * plus 16 rows of the shadow) runs in smaller chunks. The first call per
 * (device, shape) creates hipBLASLt state (it allocates: not under graph
 * capture); later calls allocate nothing. */
uint64_t venturi_row_dense_workspace_bytes(int tokens, int n, int k);
int venturi_row_dense_run(const void* x, const void* codes, const void* high, const void* scales, void* out,
                          int tokens, int n, int k, int padded, int bits, int dtype, void* workspace,
                          uint64_t workspace_bytes, void* stream);

/* The dense bridge of the reference's native runtime (ChunkedDense chunks and
 * dequant-resident shadows): out[t][n] = x[t][k] * w[n][k]^T, dtype of the
 * plan 0 fp16 / 1 bf16 / 2 fp32, fp32 arithmetic, workspace (non-null) used as
 * the GEMM's scratch; x, w, out and workspace 16-byte aligned (the reference's
 * cuBLAS bridge takes any address; its runtime passes allocations). create
 * returns NULL with a message for another dtype.
 * hipBLASLt in place of cuBLAS; the first run per (device, shape, dtype,
 * workspace size) creates its algorithm (allocates: not under graph capture).
 * Replaces ops_api.h:21-24 / blocks.cu:674-713. */
void* venturi_dense_create(int dtype);
void venturi_dense_destroy(void* plan);
int venturi_dense_run(void* plan, const void* x, const void* w, void* out, int tokens, int n, int k, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Extension: the Q8 A16 projection in the same dense form, for prefill. The
 * contract scales each exact group dot, so each weight row is decoded to the
 * exact two-term fp16 form q*s = hi + lo (hi = fp16(q*s)), x is doubled to
 * [x | x] and one hipBLASLt GEMM over 2k columns sums the exact products in
 * fp32: outputs agree with venturi_q8_head_run to fp32 association, like the
 * matrix-core routes. Scales must be below 516 (rows with larger ones give NaN
 * outputs); fp16 activations, 1..65535 tokens, k % 8 == 0, n % 8 == 0; x and
 * out 16-byte aligned, codes 8-byte, workspace 256-byte aligned; workspace of
 * venturi_q8_dense_workspace_bytes (hipBLASLt's 32 MiB, the doubled x, and the
 * shadow of up to 8192 rows; a smaller one runs smaller chunks). First call
 * per (device, shape) as for venturi_row_dense_run. No counterpart in the
 * reference (its Q8 prefill runs the head kernel). */
uint64_t venturi_q8_dense_workspace_bytes(int tokens, int n, int k);
int venturi_q8_dense_run(const void* x, const int8_t* codes, const void* scales, void* out, int tokens, int n, int k,
                         int padded, int dtype, void* workspace, uint64_t workspace_bytes, void* stream);

/* Extension: workspace bytes of venturi_moe_q4_run (0 on invalid geometry). */
uint64_t venturi_moe_q4_bytes(int tokens, int top_k, int experts, int hidden, int inter);

/* Extension: routed-expert Q4 W4A16 MoE, replacing the per-expert host loop of
 * flash_next_moe.py:139-161 / flash_next_q4.py:204-224. x fp16 [tokens][hidden];
 * ids int64 [tokens][top_k]; scores fp16 [tokens][top_k]; gate_up planes stacked
 * [experts][2*inter][...] (gate rows first), down planes [experts][hidden][...],
 * both in the tiled layout built by moe.Q4ExpertBank.upload (128-row x
 * 256-column tiles, gate/up rows paired per wave, nibbles stored as q + 8);
 * out fp16 [tokens][hidden]; workspace 256-byte aligned. Ids outside
 * [0, experts) are skipped and counted in the workspace status word, and the
 * tokens that carry one get rows of NaN (no host synchronisation). */
int venturi_moe_q4_run(const void* x, const int64_t* ids, const void* scores, const void* gate_up_codes,
                       const void* gate_up_scales, const void* down_codes, const void* down_scales, void* out,
                       void* workspace, uint64_t workspace_bytes, int tokens, int top_k, int experts, int hidden,
                       int inter, void* stream);

/* Elementwise SwiGLU out = cast((a * sigmoid(a)) * b) with fp32 math and one
 * rounding, and add out = cast(a + b); dtype 0/1/2. Replaces blocks.cu:741-750
 * (ops_api.h). */
int venturi_swiglu_run(const void* a, const void* b, void* out, int64_t count, int dtype, void* stream);
int venturi_add_run(const void* a, const void* b, void* out, int64_t count, int dtype, void* stream);

/* Extension: the same SwiGLU over one fused gate+up output [tokens][2*inter]
 * (gate columns first) -> out [tokens][inter]; dtype 0 (fp16) or 1 (bf16). */
int venturi_silu_mul_run(const void* gate_up, void* out, int tokens, int inter, int dtype, void* stream);

/* ---- Native-runtime plan table and per-matrix dispatch (no exported
 * counterpart in the reference: its runtime compiles rowcodec::prepare,
 * row_codec_dispatch.cuh:6-64, and Model::project, qwen_runtime.cuh:348-390,
 * into the model). ---- */

/* A QuantLinear plan: codec (bits, group), precision 0 = WxA16, 1 = WxA8,
 * 2 = WxA8 with the residual pass; dtype 0 fp16 / 1 bf16; implementation
 * 0 = auto, 1 = dequant, 2 = fused research; path 0 = direct, 1 = chunked
 * dense (the W*A16 contract), 2 = quantized (A8); passes = A8 passes. */
typedef struct VRCPlan {
    int bits, group, precision, dtype, implementation, path, passes;
} VRCPlan;

/* rowcodec::prepare for gfx950: fills `plan` or returns -1 with a message
 * when no kernel family is admitted (q8_g32 Auto only, A8 fp16 only; q4/q5/q6
 * fp16 WxA16 only; fused research for q4 only). */
int venturi_rowcodec_prepare(int bits, int group, int precision, int dtype, int implementation, VRCPlan* plan);

/* Workspace of venturi_rowcodec_project for `tokens` rows of K = k: the A8
 * activation pack for quantized plans (venturi_q8_dp4a_bytes); for fp16
 * ChunkedDense plans at 1024 tokens or more, the dense route's fixed buffer
 * (224 MiB: hipBLASLt's 32 MiB and the fp16 shadow, see venturi_row_dense_run;
 * with less, those plans run the fused matrix-core GEMM); 0 otherwise (and 0
 * with a message for an invalid plan). */
uint64_t venturi_rowcodec_workspace_bytes(const VRCPlan* plan, int tokens, int k);

/* One matrix of Model::project: out [tokens][n] = x [tokens][k] times the
 * row-split planes (codes, q5/q6 `high`, scales). Quantized plans quantize x
 * into `workspace` first unless `packed` = 1 (the caller filled it). */
int venturi_rowcodec_project(const VRCPlan* plan, const void* x, const void* codes, const void* high,
                             const void* scales, void* out, void* workspace, uint64_t available, int tokens, int n,
                             int k, int padded, int packed, void* stream);

/* ---- Reference exports outside the quantized-linear path. The reference's
 * Python backend binds each of these when it is constructed
 * (blocks.py:336-427), so they are exported with the reference's signatures;
 * every call returns -1 with the message "<name>: not built for gfx950
 * (outside the quantized-linear path)", makes no HIP call and writes nothing. ---- */

/* ops_api.h:46-47 */
int venturi_greedy_run(const void* logits, int64_t* out, void* workspace, size_t workspace_bytes, int rows,
                       int vocab, int dtype, void* stream);
/* ops_api.h:30-31 */
int venturi_fp32_linear_run(const void* x, const float* w, void* out, int tokens, int n, int k, int dtype,
                            void* stream);
/* ops_api.h:95-96 */
int venturi_rope_run(const void* x, const float* cos, const float* sin, void* out, int tokens, int heads, int d,
                     int r, int interleaved, int dtype, void* stream);
/* ops_api.h:87-90 */
int venturi_qwen_qk_run(const void* qg, const void* key, const float* qgamma, const float* kgamma, const float* cos,
                        const float* sin, void* qout, void* kout, int tokens, int hq, int hkv, int d, int r,
                        int dtype, float epsilon, void* stream);
/* ops_api.h:85-86 */
int venturi_qwen_gate_run(const void* x, const void* qg, void* out, int tokens, int heads, int d, int dtype,
                          void* stream);
/* ops_api.h:13-15 */
int venturi_attention_run(const void* q, const void* k, const void* v, void* out, int tokens, int kv_tokens, int hq,
                          int hkv, int d, int dtype, float scale, void* stream);
/* ops_api.h:28-29 */
int venturi_embedding_run(const void* weight, const int64_t* ids, void* out, int tokens, int vocab, int hidden,
                          int dtype, void* stream);
/* ops_api.h:42-44 */
int venturi_gdn_run(const void* q, const void* k, const void* v, const float* g, const float* beta,
                    const float* state, void* out, float* state_out, int tokens, int hqk, int hv, int dk, int dv,
                    int normalize, int packed, int dtype, float scale, void* stream);
/* ops_api.h:19-20 */
int venturi_conv_run(const void* x, const void* w, const void* history, void* out, void* history_out, int tokens,
                     int channels, int kernel, int dtype, int fp32_weight, void* stream);
/* ops_api.h:34-35 */
int venturi_gates_run(const void* a, const void* b, const float* rate, const float* bias, float* g, float* beta,
                      int tokens, int heads, int dtype, int round_beta, void* stream);
/* ops_api.h:32-33 */
int venturi_gated_rms_run(const void* x, const void* z, const void* w, void* out, int tokens, int heads,
                          int features, int dtype, int fp32_weight, float epsilon, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VENTURI_OPS_H */
