// FP8 (e4m3fn) block-scaled weight GEMM for gfx950: the C entry points over the byte-weight
// GEMM of byte_weight_gemm.h with the e4m3 decoder.
//
// Semantics (reference tasks/fp8_microscale/fp8_microscale__llama3_8b_down__b128__fp16/
// environment/reference.py:9-12):
//   W[k, n] = dtype(fp32(w_fp8[k, n]) * fp32(scales[k/B, n]))     (scales fp16, one rounding)
//   y       = x @ W                                                (x, y in fp16 or bf16)
// Dequantization is exact to the reference: gfx950's v_cvt_scalef32_pk_{f16,f32}_fp8 decode OCP
// e4m3 exactly (scale 1.0), the fp16 x fp16 product is rounded once by v_pk_mul_f16 (for bf16
// the fp32 product is exact and rounded once to bf16).
#include "byte_weight_gemm.h"

extern "C" size_t kbh_fp8w_workspace_bytes(int M, int N, int K, int block) {
  (void)block;
  kbh::BytePlan p;
  if (M < 1 || N < 128 || K < 32 || !kbh::plan_byte_decode(M, N, K, &p)) return 0;
  return kbh::splitk_workspace_bytes(M, N, p.splits);
}

extern "C" int kbh_fp8w_gemm(const void* x, const uint8_t* w_fp8, const void* scales, void* y,
                             void* workspace, size_t workspace_bytes, int M, int N, int K,
                             int block, int dtype, void* stream) {
  using namespace kbh;
  if (!x || !w_fp8 || !scales || !y) return KBH_ERR_NULL;
  if (dtype != KBH_F16 && dtype != KBH_BF16) return KBH_ERR_DTYPE;
  if (M < 1 || N < 128 || (N % 128) != 0 || K < 32 || (K % 32) != 0) return KBH_ERR_SHAPE;
  if (block != 32 && block != 64 && block != 128 && block != 256) return KBH_ERR_SHAPE;
  if (K % block != 0) return KBH_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w_fp8) || !aligned16(scales) || !aligned16(y)) return KBH_ERR_ALIGN;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == KBH_BF16)
    return byte_gemm_run<true, kDecE4M3>(x, w_fp8, scales, y, workspace, workspace_bytes, M, N, K, block, st);
  return byte_gemm_run<false, kDecE4M3>(x, w_fp8, scales, y, workspace, workspace_bytes, M, N, K, block, st);
}
