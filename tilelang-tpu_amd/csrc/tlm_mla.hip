// MLA paged decode (FP8 / fp16 / bf16 latent KV) and the paged-gather integer-path check.
#include "tlm_common.h"

namespace {

// ------------------------------------------------------------------------------------------------
// Paged gather: one 64-lane wave per token row; rows resolved through the block table exactly
// as the decode kernel resolves them (examples/deepseek_mla/example_mla_decode_paged.py:62-63).
__global__ __launch_bounds__(256) void paged_gather_kernel(
    const uint8_t* __restrict__ kv, int64_t row_bytes, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ seqlens, const int64_t* __restrict__ cu, uint8_t* __restrict__ out,
    int64_t page, int64_t max_pages) {
  const int b = blockIdx.y;
  const int64_t L = seqlens[b];
  const int lane = threadIdx.x & 63;
  for (int64_t j = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); j < L; j += (int64_t)gridDim.x * 4) {
    const int64_t row = (int64_t)block_table[b * max_pages + j / page] * page + j % page;
    const uint8_t* src = kv + row * row_bytes;
    uint8_t* dst = out + (cu[b] + j) * row_bytes;
    for (int64_t c = lane; c < row_bytes; c += 64) dst[c] = src[c];
  }
}

}  // namespace

extern "C" size_t tlm_mla_workspace_bytes(int64_t B, int64_t Hq, int64_t dv, int num_split) {
  if (B <= 0 || Hq <= 0 || dv <= 0 || num_split <= 0) return 0;
  // partial outputs fp32 [B, Hq, ns, dv] + log2-sum-exp fp32 [B, Hq, ns]
  return (size_t)B * Hq * num_split * (dv + 1) * sizeof(float);
}

extern "C" int tlm_mla_decode(const void* q, const void* q_pe, int64_t q_stride,
                              int64_t q_pe_stride, const void* kv, const void* k_pe,
                              int64_t kv_stride, int64_t kpe_stride, const int32_t* block_table,
                              const int32_t* seqlens, void* o, void* ws, size_t ws_bytes,
                              int64_t B, int64_t Hq, int64_t dv, int64_t dpe, int64_t page,
                              int64_t max_pages, int num_split, float sm_scale,
                              const float* kv_scale, int q_dtype, int kv_dtype, int o_dtype,
                              void* stream) {
  if (!q || !q_pe || !kv || !k_pe || !block_table || !seqlens || !o) {
    tlm_set_error("tlm_mla_decode: null pointer argument");
    return TLM_EINVAL;
  }
  if (B < 0 || Hq <= 0 || page <= 0 || max_pages <= 0 || num_split <= 0 || num_split > 64) {
    tlm_set_error("tlm_mla_decode: bad sizes B=%lld Hq=%lld page=%lld max_pages=%lld splits=%d",
                  (long long)B, (long long)Hq, (long long)page, (long long)max_pages, num_split);
    return TLM_EINVAL;
  }
  if (dv != 512 || dpe != 64 || Hq % 64 != 0) {
    tlm_set_error("tlm_mla_decode: kernels exist for dv=512, dpe=64, Hq a multiple of 64 "
                  "(got dv=%lld dpe=%lld Hq=%lld)", (long long)dv, (long long)dpe, (long long)Hq);
    return TLM_EUNSUPPORTED;
  }
  if (q_stride < dv || q_pe_stride < dpe || kv_stride < dv || kpe_stride < dpe) {
    tlm_set_error("tlm_mla_decode: row strides smaller than the row widths");
    return TLM_EINVAL;
  }
  if (ws_bytes < tlm_mla_workspace_bytes(B, Hq, dv, num_split) || (B > 0 && !ws)) {
    tlm_set_error("tlm_mla_decode: workspace of %zu bytes is smaller than the %zu required",
                  ws_bytes, tlm_mla_workspace_bytes(B, Hq, dv, num_split));
    return TLM_EWORKSPACE;
  }
  if ((q_dtype != TLM_BF16 && q_dtype != TLM_F16) || (o_dtype != TLM_BF16 && o_dtype != TLM_F16) ||
      (kv_dtype != TLM_F8E4M3 && kv_dtype != TLM_BF16 && kv_dtype != TLM_F16)) {
    tlm_set_error("tlm_mla_decode: dtype combination q=%d kv=%d o=%d unsupported", q_dtype,
                  kv_dtype, o_dtype);
    return TLM_EUNSUPPORTED;
  }
  if (B == 0) return TLM_OK;
  (void)sm_scale;
  (void)kv_scale;
  (void)stream;
  tlm_set_error("tlm_mla_decode: kernel not built yet");
  return TLM_EUNSUPPORTED;
}

extern "C" int tlm_paged_gather(const void* kv_bytes, int64_t row_bytes,
                                const int32_t* block_table, const int32_t* seqlens,
                                const int64_t* cu_seqlens, void* out, int64_t B, int64_t page,
                                int64_t max_pages, void* stream) {
  if (!kv_bytes || !block_table || !seqlens || !cu_seqlens || !out) {
    tlm_set_error("tlm_paged_gather: null pointer argument");
    return TLM_EINVAL;
  }
  if (B < 0 || B > 65535 || row_bytes <= 0 || page <= 0 || max_pages <= 0) {
    tlm_set_error("tlm_paged_gather: bad sizes");
    return TLM_EINVAL;
  }
  if (B == 0) return TLM_OK;
  dim3 grid(256, (unsigned)B);
  paged_gather_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)kv_bytes, row_bytes, block_table, seqlens, cu_seqlens, (uint8_t*)out, page,
      max_pages);
  TLM_LAUNCH_CHECK("tlm_paged_gather");
  return TLM_OK;
}
