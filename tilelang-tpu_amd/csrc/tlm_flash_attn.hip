// FlashAttention forward (BSHD) on MFMA.
#include "tlm_common.h"

extern "C" int tlm_flash_attn_fwd(const void* q, const void* k, const void* v, void* o,
                                  int64_t B, int64_t S, int64_t H, int64_t D, int causal,
                                  float sm_scale, int dtype, void* stream) {
  if (!q || !k || !v || !o) {
    tlm_set_error("tlm_flash_attn_fwd: null pointer argument");
    return TLM_EINVAL;
  }
  if (B < 0 || S < 0 || H < 0 || B > 65535 || H > 65535 || S > INT32_MAX) {
    tlm_set_error("tlm_flash_attn_fwd: bad shape");
    return TLM_EINVAL;
  }
  if (D != 128 && D != 64) {
    tlm_set_error("tlm_flash_attn_fwd: head dim %lld unsupported (64 or 128)", (long long)D);
    return TLM_EUNSUPPORTED;
  }
  if (dtype != TLM_BF16 && dtype != TLM_F16) {
    tlm_set_error("tlm_flash_attn_fwd: dtype %d unsupported (BF16 or F16)", dtype);
    return TLM_EUNSUPPORTED;
  }
  if (B == 0 || S == 0 || H == 0) return TLM_OK;
  (void)causal;
  (void)sm_scale;
  (void)stream;
  tlm_set_error("tlm_flash_attn_fwd: kernel not built yet");
  return TLM_EUNSUPPORTED;
}
