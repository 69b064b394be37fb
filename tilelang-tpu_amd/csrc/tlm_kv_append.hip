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
// HBM-bound streaming kernel: one thread per VEC elements (VEC = 16: two 16-byte loads, one
// 16-byte store; VEC = 8 when D or the cache's row stride is not a multiple of 16), grid-stride
// over all (sequence, token, chunk) triples, at most 4096 workgroups. The source rows are read
// once, with non-temporal loads (6% faster per launch than plain loads on HBM-resident inputs).
// (One wave per token row, or four rows per wave with their loads issued together, measured
// 10-20% slower.)
#include "tlm_common.h"

namespace {

// Cache policy of the fp8 page stores (st_cp) when the pool spans less than 2^31 bytes (buffer
// offsets from the pool base); larger pools store through plain global stores.
constexpr int kKvStoreCP = CP_NT;
constexpr int kKvLoadCP = CP_GLOBAL_NT;  // the source rows (read once)
// Launch shape, measured on the B 64, T 512, D 576 bf16 chunk (back to back): 256 threads and one
// row group per thread (4,736 workgroups) 4.48 TB/s; two or four row groups per thread with their
// loads issued together 3.68 / 3.40 TB/s; 128 / 64 / 512 threads 4.31-4.37 / 3.93 / 4.31 TB/s.
constexpr int kKvWgCap = 8192;  // workgroups per launch at most
constexpr int KV_U = 1;         // row groups per thread and iteration (loads issued together)
constexpr int KV_T = 256;       // threads per workgroup

// One workgroup handles `rows` token rows of one sequence at a time (blockIdx.y strides over the
// sequences, so start[b] / count[b] are uniform loads): thread t owns chunk t % chunks of row
// t / chunks, both fixed for the whole loop; rows longer than 256 chunks loop over chunks with
// one row per workgroup. page_shift >= 0: the page size is 2^page_shift (shift and mask instead
// of a 64-bit division).
template <bool BF16, int VEC, bool BUF>
__global__ __launch_bounds__(KV_T) void kv_append_fp8_kernel(
    const uint16_t* __restrict__ x, int64_t x_bstride, int64_t x_rstride,
    const int32_t* __restrict__ start, const int32_t* __restrict__ count,
    const int32_t* __restrict__ block_table, int64_t max_pages, int64_t page, int page_shift,
    uint8_t* __restrict__ kv, int64_t kv_stride, int64_t kv_rows, int B, int T, int chunks,
    int rows, const float* __restrict__ scale) {
  using H = h16<BF16>;
  const float s = *scale;
  // x / s correctly rounded without a division per element (Markstein): with y = RN(1 / s),
  // q0 = RN(x y) and r = x - q0 s (exact in an fma), RN(q0 + r y) = RN(x / s) whenever the
  // residual does not underflow, which holds for |x| >= 2^-100 (checked against exact quotients
  // over 1.5e8 random pairs). For 2^-90 <= s <= 2^90 every smaller |x| gives |x / s| < 2^-10,
  // which rounds to a signed e4m3 zero whatever the last fp32 bit, so the uniform fast path
  // needs no per-element guard: q0 is clamped to +-1024 before the refinement so an overflowing
  // x y cannot turn into inf - inf, the sign is taken from q0 (an fma of a zero residual drops
  // the sign of -0), and NaN inputs are passed through. Other scales divide per element.
  const float y = __fdiv_rn(1.0f, s);
  const bool fast = s >= 0x1p-90f && s <= 0x1p90f;
  const int r = (int)threadIdx.x / chunks;  // row of the group (0 when chunks > KV_T)
  const int c0 = (int)threadIdx.x - r * chunks;
  if (r >= rows) return;  // threads past the last whole row (no barriers in this kernel)
  const int64_t pool_tokens = max_pages * page;

  auto load = [&](int b, int j, int c, u32x4 (&w)[VEC / 8]) {
    const u32x4* src = (const u32x4*)(x + b * x_bstride + j * x_rstride + VEC * c);
#pragma unroll
    for (int u = 0; u < VEC / 8; ++u) w[u] = ld_cp<kKvLoadCP>(src, 16 * u);  // read once
  };
  auto convert = [&](const u32x4 (&w)[VEC / 8], int c, int64_t row) {
    float v[VEC];
#pragma unroll
    for (int u = 0; u < VEC / 8; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[8 * u + 2 * e] = H::lo(w[u][e]);
        v[8 * u + 2 * e + 1] = H::hi(w[u][e]);
      }
    if (fast) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float q0 = v[e] * y;
        const float qc = __builtin_amdgcn_fmed3f(q0, -1024.f, 1024.f);
        const float q1 = copysignf(fmaf(fmaf(-qc, s, v[e]), y, qc), q0);
        const float o = __builtin_amdgcn_fmed3f(q1, -448.f, 448.f);  // saturate
        v[e] = v[e] != v[e] ? v[e] : o;                                // NaN stays NaN
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float q = __fdiv_rn(v[e], s);
        v[e] = q != q ? q : fminf(fmaxf(q, -448.f), 448.f);
      }
    }
    // v_cvt_pk_fp8_f32 rounds to nearest even (448 is the largest finite e4m3; a 464 tie rounds
    // to it, larger magnitudes would give the NaN code, hence the clamp above).
    uint32_t o[VEC / 4];
#pragma unroll
    for (int h = 0; h < VEC / 4; ++h) {
      int word = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * h], v[4 * h + 1], 0, false);
      word = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * h + 2], v[4 * h + 3], word, true);
      o[h] = (uint32_t)word;
    }
    uint8_t* dst = kv + row * kv_stride + VEC * c;
    if constexpr (VEC == 16 && BUF) {
      st_cp<kKvStoreCP>(kv, (int)(row * kv_stride + VEC * c), u32x4{o[0], o[1], o[2], o[3]});
    } else if constexpr (VEC == 16) {
      *(u32x4*)dst = u32x4{o[0], o[1], o[2], o[3]};
    } else {
      *(u32x2*)dst = u32x2{o[0], o[1]};
    }
  };

  for (int b = blockIdx.y; b < B; b += gridDim.y) {
    const int cnt = min(count[b], T);
    const int64_t st = start[b];
    const int step = gridDim.x * rows;
    for (int j0 = blockIdx.x * rows + r; j0 < cnt; j0 += step * KV_U) {
      // the source rows exist for every j < cnt: their loads (KV_U rows, step apart) go out
      // before the table lookups, so the global reads overlap instead of running back to back
      u32x4 w[KV_U][VEC / 8];
#pragma unroll
      for (int u = 0; u < KV_U; ++u)
        if (j0 + u * step < cnt) load(b, j0 + u * step, c0, w[u]);
#pragma unroll
      for (int u = 0; u < KV_U; ++u) {
        const int j = j0 + u * step;
        if (j >= cnt) break;
        const int64_t p = st + j;
        if (p < 0 || p >= pool_tokens) continue;  // beyond the block table
        const int64_t pg = page_shift >= 0 ? p >> page_shift : p / page;
        const int64_t off = page_shift >= 0 ? p & (page - 1) : p % page;
        const int64_t row = (int64_t)block_table[b * max_pages + pg] * page + off;
        if (row < 0 || row >= kv_rows) continue;  // a corrupt table entry never writes out of the pool
        convert(w[u], c0, row);
        for (int c = c0 + KV_T; c < chunks; c += KV_T) {  // rows of more than KV_T chunks
          load(b, j, c, w[u]);
          convert(w[u], c, row);
        }
      }
    }
  }
}

template <bool BF16, int VEC>
void launch(const void* x, int64_t xb, int64_t xr, const int32_t* start, const int32_t* count,
            const int32_t* bt, int64_t max_pages, int64_t page, void* kv, int64_t kv_stride,
            int64_t kv_rows, int64_t B, int64_t T, int64_t D, const float* scale, hipStream_t st) {
  const int chunks = (int)(D / VEC);
  const int rows = chunks > KV_T ? 1 : KV_T / chunks;  // token rows per workgroup
  int shift = -1;
  if ((page & (page - 1)) == 0) shift = __builtin_ctzll((unsigned long long)page);
  const int64_t gy = std::min<int64_t>(B, 65535);
  const int64_t gx =
      std::min<int64_t>((T + rows * KV_U - 1) / (rows * KV_U), std::max<int64_t>(1, kKvWgCap / gy));
  const dim3 grid((unsigned)gx, (unsigned)gy);
  auto go = [&](auto kern) {
    kern<<<grid, KV_T, 0, st>>>((const uint16_t*)x, xb, xr, start, count, bt, max_pages, page,
                               shift, (uint8_t*)kv, kv_stride, kv_rows, (int)B, (int)T, chunks,
                               rows, scale);
  };
  if (kv_rows * kv_stride < ((int64_t)1 << 31))  // buffer offsets from the pool base fit
    go(kv_append_fp8_kernel<BF16, VEC, true>);
  else
    go(kv_append_fp8_kernel<BF16, VEC, false>);
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
  if (B * T * (D / 8) > INT32_MAX || B * max_pages > INT32_MAX) {
    tlm_set_error("tlm_kv_append_fp8: problem too large for one launch");
    return TLM_EINVAL;
  }
  hipStream_t st = (hipStream_t)stream;
  const bool v16 = D % 16 == 0 && kv_stride % 16 == 0 && tlm_aligned(kv, 16);
  if (x_dtype == TLM_BF16) {
    if (v16)
      launch<true, 16>(x, x_batch_stride, x_row_stride, start, count, block_table, max_pages,
                       page, kv, kv_stride, kv_rows, B, T, D, scale, st);
    else
      launch<true, 8>(x, x_batch_stride, x_row_stride, start, count, block_table, max_pages,
                      page, kv, kv_stride, kv_rows, B, T, D, scale, st);
  } else {
    if (v16)
      launch<false, 16>(x, x_batch_stride, x_row_stride, start, count, block_table, max_pages,
                        page, kv, kv_stride, kv_rows, B, T, D, scale, st);
    else
      launch<false, 8>(x, x_batch_stride, x_row_stride, start, count, block_table, max_pages,
                       page, kv, kv_stride, kv_rows, B, T, D, scale, st);
  }
  TLM_LAUNCH_CHECK("tlm_kv_append_fp8");
  return TLM_OK;
}
