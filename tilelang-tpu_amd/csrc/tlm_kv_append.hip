// Paged KV-cache append with FP8 (OCP e4m3) quantisation: the step before the FP8 MLA decode.
//
// New latent rows (bf16 / fp16) are scaled by the cache's per-tensor scale, quantised to e4m3 and
// written into their pages through the block table. The page address of token position p of
// sequence b is block_table[b, p / page] * page + p % page, the same addressing the decode reads
// (examples/deepseek_mla/example_mla_decode_paged.py:62-63, block table layout :26).
//
// Quantisation: q = e4m3(clamp(x / scale, -448, 448)) with x / scale correctly rounded in fp32
// and one round-to-nearest-even into e4m3 (v_cvt_pk_fp8_f32); NaN stays NaN. Inside [-448, 448]
// this is exactly torch's (x.float() / scale).to(torch.float8_e4m3fn), which is how the MLA
// config's cache is built; out-of-range values saturate instead of becoming NaN.
//
// HBM-bound streaming kernel: one thread per 8 elements (one 16-byte load, one 8-byte store),
// grid-stride over all (sequence, token, chunk) triples. (One wave per token row, or four rows
// per wave with their loads issued together, measured 10-15% slower at the bench size.)
#include "tlm_common.h"

namespace {

template <bool BF16>
__global__ __launch_bounds__(256) void kv_append_fp8_kernel(
    const uint16_t* __restrict__ x, int64_t x_bstride, int64_t x_rstride,
    const int32_t* __restrict__ start, const int32_t* __restrict__ count,
    const int32_t* __restrict__ block_table, int64_t max_pages, int64_t page,
    uint8_t* __restrict__ kv, int64_t kv_stride, int64_t kv_rows, int T, int chunks, int total,
    const float* __restrict__ scale) {
  using H = h16<BF16>;
  const float s = *scale;
  // x / s correctly rounded without a division per element (Markstein): y = RN(1 / s),
  // q = RN(x y), q' = RN(q + RN(x - q s) y) is RN(x / s) when the residual does not underflow
  // (|x| >= 2^-100; checked against exact quotients over 1.5e8 random pairs); zeros keep their
  // sign through q, quotients beyond 1e30 saturate anyway, tiny x takes the division.
  const float y = __fdiv_rn(1.0f, s);
  for (int i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
    const int c = i % chunks;
    const int bt = i / chunks;
    const int b = bt / T, j = bt % T;
    if (j >= count[b]) continue;
    const int64_t p = (int64_t)start[b] + j;
    if (p < 0 || p >= max_pages * page) continue;  // beyond the block table
    const int64_t row = (int64_t)block_table[b * max_pages + p / page] * page + p % page;
    if (row < 0 || row >= kv_rows) continue;  // a corrupt table entry never writes out of the pool
    const u32x4 w = *(const u32x4*)(x + b * x_bstride + j * x_rstride + 8 * c);
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = H::lo(w[e]);
      v[2 * e + 1] = H::hi(w[e]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float ax = fabsf(v[e]);
      float q = v[e] * y;
      if (ax >= 0x1p-100f && fabsf(q) <= 1e30f)
        q = fmaf(fmaf(-q, s, v[e]), y, q);
      else if (ax != 0.f && ax < 0x1p-100f)
        q = __fdiv_rn(v[e], s);
      v[e] = q != q ? q : fminf(fmaxf(q, -448.f), 448.f);  // saturate, keep NaN
    }
    u32x2 o;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int word = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * h], v[4 * h + 1], 0, false);
      word = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * h + 2], v[4 * h + 3], word, true);
      o[h] = (uint32_t)word;
    }
    *(u32x2*)(kv + row * kv_stride + 8 * c) = o;
  }
}

}  // namespace

extern "C" int tlm_kv_append_fp8(const void* x, int64_t x_batch_stride, int64_t x_row_stride,
                                 int x_dtype, const int32_t* start, const int32_t* count,
                                 const int32_t* block_table, int64_t max_pages, int64_t page,
                                 void* kv, int64_t kv_stride, int64_t kv_rows, int64_t B,
                                 int64_t T, int64_t D, const float* scale, void* stream) {
  if (!x || !start || !count || !block_table || !kv || !scale) {
    tlm_set_error("tlm_kv_append_fp8: null pointer argument");
    return TLM_EINVAL;
  }
  if (B < 0 || T < 0 || D <= 0 || page <= 0 || max_pages <= 0 || kv_rows < 0 ||
      x_batch_stride < 0 || x_row_stride < 0 || kv_stride < D) {
    tlm_set_error("tlm_kv_append_fp8: bad sizes");
    return TLM_EINVAL;
  }
  if (x_dtype != TLM_BF16 && x_dtype != TLM_F16) {
    tlm_set_error("tlm_kv_append_fp8: x dtype %d unsupported (BF16 or F16)", x_dtype);
    return TLM_EUNSUPPORTED;
  }
  if (D % 8 != 0 || x_row_stride % 8 != 0 || x_batch_stride % 8 != 0 || kv_stride % 8 != 0) {
    tlm_set_error("tlm_kv_append_fp8: D and strides must be multiples of 8 elements");
    return TLM_EUNSUPPORTED;
  }
  if (!tlm_aligned(x, 16) || !tlm_aligned(kv, 8)) {
    tlm_set_error("tlm_kv_append_fp8: x must be 16-byte and kv 8-byte aligned");
    return TLM_EINVAL;
  }
  if (B == 0 || T == 0) return TLM_OK;
  const int64_t chunks = D / 8;
  if (B * T * chunks > INT32_MAX || B * max_pages > INT32_MAX) {
    tlm_set_error("tlm_kv_append_fp8: problem too large for one launch");
    return TLM_EINVAL;
  }
  const int total = (int)(B * T * chunks);
  const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 256 * 16);
  hipStream_t st = (hipStream_t)stream;
  if (x_dtype == TLM_BF16)
    kv_append_fp8_kernel<true><<<grid, 256, 0, st>>>(
        (const uint16_t*)x, x_batch_stride, x_row_stride, start, count, block_table, max_pages,
        page, (uint8_t*)kv, kv_stride, kv_rows, (int)T, (int)chunks, total, scale);
  else
    kv_append_fp8_kernel<false><<<grid, 256, 0, st>>>(
        (const uint16_t*)x, x_batch_stride, x_row_stride, start, count, block_table, max_pages,
        page, (uint8_t*)kv, kv_stride, kv_rows, (int)T, (int)chunks, total, scale);
  TLM_LAUNCH_CHECK("tlm_kv_append_fp8");
  return TLM_OK;
}
