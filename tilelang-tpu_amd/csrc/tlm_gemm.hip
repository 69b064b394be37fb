// GEMM C = A * B on MFMA (fp16 / bf16 in, fp32 accumulate).
#include "tlm_common.h"

extern "C" int tlm_gemm(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                        int in_dtype, int out_dtype, int trans_b, void* stream) {
  if (!A || !B || !C) {
    tlm_set_error("tlm_gemm: null pointer argument");
    return TLM_EINVAL;
  }
  if (M < 0 || N < 0 || K < 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) {
    tlm_set_error("tlm_gemm: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                  (long long)K);
    return TLM_EINVAL;
  }
  if (trans_b != 0 && trans_b != 1) {
    tlm_set_error("tlm_gemm: trans_b must be 0 or 1");
    return TLM_EINVAL;
  }
  if (in_dtype != TLM_F16 && in_dtype != TLM_BF16) {
    tlm_set_error("tlm_gemm: in_dtype %d unsupported (F16 or BF16)", in_dtype);
    return TLM_EUNSUPPORTED;
  }
  if (out_dtype != TLM_F16 && out_dtype != TLM_BF16 && out_dtype != TLM_F32) {
    tlm_set_error("tlm_gemm: out_dtype %d unsupported", out_dtype);
    return TLM_EUNSUPPORTED;
  }
  if (M == 0 || N == 0) return TLM_OK;
  (void)stream;
  tlm_set_error("tlm_gemm: kernel not built yet");
  return TLM_EUNSUPPORTED;
}
