/*
 * C restatement of the byte/integer parts of the kernel path. TEST INFRASTRUCTURE ONLY:
 * loaded by tests/ (and usable by the CPU baseline) as a checker, never by the product.
 *
 *  - oracle_fp8_e4m3fn_decode: OCP e4m3fn -> float (bias 7, 3 mantissa bits, subnormals at
 *    exponent 0, 0x7F/0xFF NaN, no infinities). The MLA config stores its KV cache in this
 *    format; the reference's MLA oracle dequantises implicitly via
 *    torch (examples/deepseek_mla/example_mla_decode_paged.py:267-270 calls .float()).
 *  - oracle_paged_gather: page addressing of the MLA kernel,
 *      row(b, j) = block_table[b, j / page] * page + j % page
 *    (examples/deepseek_mla/example_mla_decode_paged.py:62-63 and 147-148), rows copied in token
 *    order, sequences concatenated.
 *  - oracle_rmsnorm_f64: brute-force double-precision RMSNorm of float rows
 *    (tpu_demo/rms_norm/rms_norm_fp16.py:51-54 plus weight), used to pin the torch oracle.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

float oracle_fp8_e4m3fn_decode_one(uint8_t b) {
  int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
  float v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0)
    v = ldexpf((float)m, -9); /* m/8 * 2^-6 */
  else
    v = ldexpf(8.0f + (float)m, e - 10); /* (1 + m/8) * 2^(e-7) */
  return s ? -v : v;
}

void oracle_fp8_e4m3fn_decode(const uint8_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_fp8_e4m3fn_decode_one(in[i]);
}

/* Returns the number of rows written, or -1 if a row index falls outside [0, n_rows). */
int64_t oracle_paged_gather(const uint8_t* kv, int64_t row_bytes, int64_t n_rows,
                            const int32_t* block_table, const int32_t* seqlens, int64_t B,
                            int64_t max_pages, int64_t page, uint8_t* out) {
  int64_t w = 0;
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t j = 0; j < seqlens[b]; ++j) {
      int64_t p = j / page;
      if (p >= max_pages) return -1;
      int64_t row = (int64_t)block_table[b * max_pages + p] * page + j % page;
      if (row < 0 || row >= n_rows) return -1;
      memcpy(out + w * row_bytes, kv + row * row_bytes, (size_t)row_bytes);
      ++w;
    }
  }
  return w;
}

void oracle_rmsnorm_f64(const float* x, const float* w, double* y, int64_t rows, int64_t cols,
                        double eps) {
  for (int64_t r = 0; r < rows; ++r) {
    double ss = 0.0;
    for (int64_t c = 0; c < cols; ++c) ss += (double)x[r * cols + c] * (double)x[r * cols + c];
    double inv = 1.0 / sqrt(ss / (double)cols + eps);
    for (int64_t c = 0; c < cols; ++c)
      y[r * cols + c] = (double)x[r * cols + c] * inv * (w ? (double)w[c] : 1.0);
  }
}
