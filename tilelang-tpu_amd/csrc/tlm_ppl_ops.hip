// The remaining tile operations of the TPU demo programs: sigmoid, row gather, top-k (sort),
// row reductions.
//
// Reference programs and ops:
//   sigmoid    tpu_demo/tpu_test_sigmoid_fp32.py:6-31, T.ppl_sigmoid (tilelang/language/
//              customize.py:343-350, BM1690 table + polynomial, fp32 only); checked against
//              torch.sigmoid with atol = rtol = 1e-2 (:48-60).
//   gather     tpu_demo/tpu_test_gather_fp32.py:8-18, T.ppl_gather (customize.py:352-356) ->
//              tpu_gdma_h_gather_S2S (src/target/codegen_ppl.cc:1849-1877): Output[i, :] =
//              Param[Index[i], :], uint32 indices, param_h = rows of Param.
//   topk       tpu_demo/tpu_test_topk_fp32.py:6-18, T.ppl_topk (customize.py:358-362) ->
//              tpu_hau_sort_natural_index(dst, dst_idx, src, length, K, descended)
//              (codegen_ppl.cc:1878-1907): the whole vector is sorted, the first K entries are the
//              top K values and their indices; fp32 / int32 / uint32.
//   reduce     tpu_demo/tpu_test_reduce_max.py, tpu_test_reduce_sum.py: X [M, N] -> Y [M, 1]
//              row max / row sum (T.ppl_reduce_max / ppl_reduce_sum, customize.py:476-573).
//
// Stated choices where the reference leaves behaviour to the hardware:
//   * gather: an index >= param_h writes a zero row (the reference passes a 0 fill value);
//   * topk: ties are ordered by index (a stable sort), every NaN counts as larger than +inf and
//     -0.0 equals +0.0, as torch.sort(stable=True); all `length` entries are written in order;
//   * reduce_max propagates NaN (torch.max does); reduce_sum accumulates in fp32, rounds once.
#include "tlm_common.h"

namespace {

template <int DT>
TLM_DEV float ld_as_f32(const void* p, int64_t i) {
  if constexpr (DT == TLM_F32) return ((const float*)p)[i];
  else return h16<DT == TLM_BF16>::to_f32(((const uint16_t*)p)[i]);
}
template <int DT>
TLM_DEV void st_from_f32(void* p, int64_t i, float v) {
  if constexpr (DT == TLM_F32) ((float*)p)[i] = v;
  else ((uint16_t*)p)[i] = (uint16_t)h16<DT == TLM_BF16>::from_f32(v);
}

unsigned grid_for(int64_t work, int per_block, int64_t cap) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g > cap) g = cap;
  return (unsigned)(g < 1 ? 1 : g);
}

// ---- sigmoid: y = 1 / (1 + exp(-x)) in fp32, one rounding for 16-bit outputs
TLM_DEV float sigmoid1(float x) { return __builtin_amdgcn_rcpf(fast_exp(-x) + 1.0f); }

__global__ __launch_bounds__(256) void sigmoid_f32_vec(const f32x4* __restrict__ x,
                                                       f32x4* __restrict__ y, int64_t nvec) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec;
       i += (int64_t)gridDim.x * 256) {
    const f32x4 v = __builtin_nontemporal_load(x + i);
    __builtin_nontemporal_store(f32x4{sigmoid1(v[0]), sigmoid1(v[1]), sigmoid1(v[2]),
                                      sigmoid1(v[3])},
                                y + i);
  }
}

template <int DT>
__global__ __launch_bounds__(256) void sigmoid_scalar(const void* __restrict__ x,
                                                      void* __restrict__ y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256)
    st_from_f32<DT>(y, i, sigmoid1(ld_as_f32<DT>(x, i)));
}

// ---- row gather: one thread per 16-byte (or 4-byte) piece of an output row
template <typename W>
__global__ __launch_bounds__(256) void gather_rows(const W* __restrict__ param,
                                                   const uint32_t* __restrict__ index,
                                                   W* __restrict__ out, int64_t n_index,
                                                   int64_t pieces, uint32_t param_rows) {
  const int64_t total = n_index * pieces;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / pieces, c = i - r * pieces;
    const uint32_t src = index[r];
    W v;
    if (src < param_rows) {
      v = param[(int64_t)src * pieces + c];
    } else {
      v = W{};
    }
    out[i] = v;
  }
}

// ---- top-k by a bitonic sort of (key, index) pairs in LDS, one workgroup
constexpr int TOPK_THREADS = 1024;
constexpr int TOPK_MAX = 16384;  // 16384 * 8 bytes of keys and indices = 128 KB of LDS

// order-preserving unsigned key: ascending keys = ascending values; NaN above +inf; -0 == +0
template <int DT>
TLM_DEV uint32_t sort_key(uint32_t u) {
  if constexpr (DT == TLM_F32) {
    if ((u & 0x7fffffffu) > 0x7f800000u) u = 0x7fc00000u;  // every NaN alike, above +inf
    if (u == 0x80000000u) u = 0;                             // -0 == +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  } else if constexpr (DT == TLM_I32) {
    return u ^ 0x80000000u;
  } else {
    return u;
  }
}

template <int DT>
__global__ __launch_bounds__(TOPK_THREADS) void topk_bitonic(const uint32_t* __restrict__ src,
                                                             uint32_t* __restrict__ out_val,
                                                             int32_t* __restrict__ out_idx,
                                                             int length, int P, bool descending) {
  __shared__ uint32_t key[TOPK_MAX];
  __shared__ uint32_t idx[TOPK_MAX];
  for (int i = threadIdx.x; i < P; i += TOPK_THREADS) {
    if (i < length) {
      const uint32_t k = sort_key<DT>(src[i]);
      key[i] = descending ? ~k : k;
      idx[i] = (uint32_t)i;
    } else {  // padding sorts after every element
      key[i] = 0xffffffffu;
      idx[i] = 0xffffffffu;
    }
  }
  __syncthreads();
  // ascending by (key, index): lexicographic compare of the pair
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < P; i += TOPK_THREADS) {
        const int l = i ^ j;
        if (l > i) {
          const uint32_t ki = key[i], kl = key[l], ii = idx[i], il = idx[l];
          const bool up = (i & k) == 0;  // this subsequence sorts ascending
          const bool gt = ki > kl || (ki == kl && ii > il);
          if (gt == up) {
            key[i] = kl;
            key[l] = ki;
            idx[i] = il;
            idx[l] = ii;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < length; i += TOPK_THREADS) {
    const uint32_t s = idx[i];
    out_val[i] = src[s];
    out_idx[i] = (int32_t)s;
  }
}

// ---- row reductions: one wave per row, fp32 accumulation (sum) / NaN-propagating max
template <int IN, int OUT, bool MAX>
__global__ __launch_bounds__(256) void row_reduce(const void* __restrict__ x, void* __restrict__ y,
                                                  int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  float a = MAX ? -INFINITY : 0.f;
  bool nan = false;
  for (int64_t c = lane; c < cols; c += 64) {
    const float v = ld_as_f32<IN>(x, row * cols + c);
    if constexpr (MAX) {
      nan |= v != v;
      a = fmaxf(a, v);
    } else {
      a += v;
    }
  }
  if constexpr (MAX) {
    nan = __builtin_amdgcn_ballot_w64(nan) != 0;
    a = wave_max(a);
    if (nan) a = __builtin_nanf("");
  } else {
    a = wave_sum(a);
  }
  if (lane == 0) st_from_f32<OUT>(y, row, a);
}

template <int IN, bool MAX>
void launch_reduce(const void* x, void* y, int64_t rows, int64_t cols, int out, hipStream_t s) {
  const unsigned grid = (unsigned)((rows + 3) / 4);
  switch (out) {
    case TLM_F32: row_reduce<IN, TLM_F32, MAX><<<grid, 256, 0, s>>>(x, y, rows, cols); break;
    case TLM_BF16: row_reduce<IN, TLM_BF16, MAX><<<grid, 256, 0, s>>>(x, y, rows, cols); break;
    default: row_reduce<IN, TLM_F16, MAX><<<grid, 256, 0, s>>>(x, y, rows, cols); break;
  }
}

bool is_float(int dt) { return dt == TLM_F16 || dt == TLM_BF16 || dt == TLM_F32; }
int esize(int dt) { return dt == TLM_F32 || dt == TLM_I32 ? 4 : dt == TLM_F8E4M3 ? 1 : 2; }

}  // namespace

extern "C" int tlm_sigmoid(const void* x, void* y, int64_t n, int dtype, void* stream) {
  if (!x || !y) {
    tlm_set_error("tlm_sigmoid: null pointer");
    return TLM_EINVAL;
  }
  if (n < 0) {
    tlm_set_error("tlm_sigmoid: negative size");
    return TLM_EINVAL;
  }
  if (!is_float(dtype)) {
    tlm_set_error("tlm_sigmoid: dtype %d unsupported (F32, F16 or BF16)", dtype);
    return TLM_EUNSUPPORTED;
  }
  if (!tlm_aligned(x, esize(dtype)) || !tlm_aligned(y, esize(dtype))) {
    tlm_set_error("tlm_sigmoid: pointers must be aligned to the element size");
    return TLM_EINVAL;
  }
  if (n == 0) return TLM_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TLM_F32 && n % 4 == 0 && tlm_aligned(x, 16) && tlm_aligned(y, 16))
    sigmoid_f32_vec<<<grid_for(n / 4, 256, 256 * 16), 256, 0, s>>>((const f32x4*)x, (f32x4*)y,
                                                                    n / 4);
  else if (dtype == TLM_F32)
    sigmoid_scalar<TLM_F32><<<grid_for(n, 256, 256 * 16), 256, 0, s>>>(x, y, n);
  else if (dtype == TLM_BF16)
    sigmoid_scalar<TLM_BF16><<<grid_for(n, 256, 256 * 16), 256, 0, s>>>(x, y, n);
  else
    sigmoid_scalar<TLM_F16><<<grid_for(n, 256, 256 * 16), 256, 0, s>>>(x, y, n);
  TLM_LAUNCH_CHECK("tlm_sigmoid");
  return TLM_OK;
}

extern "C" int tlm_gather_rows(const void* param, int64_t param_rows, int64_t row_bytes,
                               const uint32_t* index, int64_t n_index, void* out, void* stream) {
  if (!param || !index || !out) {
    tlm_set_error("tlm_gather_rows: null pointer");
    return TLM_EINVAL;
  }
  if (param_rows < 0 || param_rows > 0xffffffffll || row_bytes <= 0 || n_index < 0 ||
      row_bytes % 2 != 0) {
    tlm_set_error("tlm_gather_rows: bad sizes (row_bytes even and positive)");
    return TLM_EINVAL;
  }
  if (!tlm_aligned(index, 4) || !tlm_aligned(param, 2) || !tlm_aligned(out, 2)) {
    tlm_set_error("tlm_gather_rows: misaligned pointer");
    return TLM_EINVAL;
  }
  if (n_index == 0) return TLM_OK;
  hipStream_t s = (hipStream_t)stream;
  const uint32_t pr = (uint32_t)param_rows;
  if (row_bytes % 16 == 0 && tlm_aligned(param, 16) && tlm_aligned(out, 16)) {
    const int64_t pieces = row_bytes / 16;
    gather_rows<u32x4><<<grid_for(n_index * pieces, 256, 256 * 16), 256, 0, s>>>(
        (const u32x4*)param, index, (u32x4*)out, n_index, pieces, pr);
  } else if (row_bytes % 4 == 0 && tlm_aligned(param, 4) && tlm_aligned(out, 4)) {
    const int64_t pieces = row_bytes / 4;
    gather_rows<uint32_t><<<grid_for(n_index * pieces, 256, 256 * 16), 256, 0, s>>>(
        (const uint32_t*)param, index, (uint32_t*)out, n_index, pieces, pr);
  } else {
    const int64_t pieces = row_bytes / 2;
    gather_rows<uint16_t><<<grid_for(n_index * pieces, 256, 256 * 16), 256, 0, s>>>(
        (const uint16_t*)param, index, (uint16_t*)out, n_index, pieces, pr);
  }
  TLM_LAUNCH_CHECK("tlm_gather_rows");
  return TLM_OK;
}

extern "C" int tlm_topk(const void* src, int64_t length, int64_t k, int descending, int dtype,
                        void* out_values, int32_t* out_indices, void* stream) {
  if (!src || !out_values || !out_indices) {
    tlm_set_error("tlm_topk: null pointer");
    return TLM_EINVAL;
  }
  if (length < 0 || k < 0 || k > length) {
    tlm_set_error("tlm_topk: need 0 <= k <= length (k=%lld, length=%lld)", (long long)k,
                  (long long)length);
    return TLM_EINVAL;
  }
  if (dtype != TLM_F32 && dtype != TLM_I32 && dtype != TLM_U32) {
    tlm_set_error("tlm_topk: dtype %d unsupported (F32, I32 or U32)", dtype);
    return TLM_EUNSUPPORTED;
  }
  if (length > TOPK_MAX) {
    tlm_set_error("tlm_topk: length %lld above the single-workgroup sort limit %d",
                  (long long)length, TOPK_MAX);
    return TLM_EUNSUPPORTED;
  }
  if (!tlm_aligned(src, 4) || !tlm_aligned(out_values, 4) || !tlm_aligned(out_indices, 4)) {
    tlm_set_error("tlm_topk: pointers must be 4-byte aligned");
    return TLM_EINVAL;
  }
  if (length == 0) return TLM_OK;
  int P = 2;
  while (P < length) P <<= 1;
  hipStream_t s = (hipStream_t)stream;
  const uint32_t* sv = (const uint32_t*)src;
  uint32_t* ov = (uint32_t*)out_values;
  if (dtype == TLM_F32)
    topk_bitonic<TLM_F32><<<1, TOPK_THREADS, 0, s>>>(sv, ov, out_indices, (int)length, P,
                                                     descending != 0);
  else if (dtype == TLM_I32)
    topk_bitonic<TLM_I32><<<1, TOPK_THREADS, 0, s>>>(sv, ov, out_indices, (int)length, P,
                                                     descending != 0);
  else
    topk_bitonic<TLM_U32><<<1, TOPK_THREADS, 0, s>>>(sv, ov, out_indices, (int)length, P,
                                                     descending != 0);
  TLM_LAUNCH_CHECK("tlm_topk");
  return TLM_OK;
}

extern "C" int tlm_row_reduce(const void* x, void* y, int64_t rows, int64_t cols, int op,
                              int in_dtype, int out_dtype, void* stream) {
  if (!x || !y) {
    tlm_set_error("tlm_row_reduce: null pointer");
    return TLM_EINVAL;
  }
  if (rows < 0 || cols <= 0 || rows > (int64_t)0xffffffff * 4) {
    tlm_set_error("tlm_row_reduce: bad shape rows=%lld cols=%lld", (long long)rows,
                  (long long)cols);
    return TLM_EINVAL;
  }
  if (op != TLM_REDUCE_MAX && op != TLM_REDUCE_SUM) {
    tlm_set_error("tlm_row_reduce: op %d unknown (TLM_REDUCE_MAX or TLM_REDUCE_SUM)", op);
    return TLM_EINVAL;
  }
  if (!is_float(in_dtype) || !is_float(out_dtype)) {
    tlm_set_error("tlm_row_reduce: dtypes %d -> %d unsupported (F32, F16, BF16)", in_dtype,
                  out_dtype);
    return TLM_EUNSUPPORTED;
  }
  if (!tlm_aligned(x, esize(in_dtype)) || !tlm_aligned(y, esize(out_dtype))) {
    tlm_set_error("tlm_row_reduce: pointers must be aligned to the element size");
    return TLM_EINVAL;
  }
  if (rows == 0) return TLM_OK;
  hipStream_t s = (hipStream_t)stream;
  const bool mx = op == TLM_REDUCE_MAX;
  switch (in_dtype) {
    case TLM_F32:
      mx ? launch_reduce<TLM_F32, true>(x, y, rows, cols, out_dtype, s)
         : launch_reduce<TLM_F32, false>(x, y, rows, cols, out_dtype, s);
      break;
    case TLM_BF16:
      mx ? launch_reduce<TLM_BF16, true>(x, y, rows, cols, out_dtype, s)
         : launch_reduce<TLM_BF16, false>(x, y, rows, cols, out_dtype, s);
      break;
    default:
      mx ? launch_reduce<TLM_F16, true>(x, y, rows, cols, out_dtype, s)
         : launch_reduce<TLM_F16, false>(x, y, rows, cols, out_dtype, s);
  }
  TLM_LAUNCH_CHECK("tlm_row_reduce");
  return TLM_OK;
}
