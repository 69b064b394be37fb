// HBM-streaming elementwise kernels: SwiGLU and interleaved RoPE.
// No MFMA and no LDS: every byte is read once with 16-byte vector loads, math in fp32, one
// rounding per output, 16-byte non-temporal stores.
#include "tlm_common.h"

namespace {

// ------------------------------------------------------------------------------------------------
// SwiGLU. Reference program tpu_demo/tpu_test_swiglu_bf16.py:5-54:
//   x = fp32(gate); e = exp(-x) (ppl_exp2 = natural exp, codegen_ppl.cc:1294-1320);
//   out = cast(up * (x / (e + 1)))   — fp32 throughout, one rounding at the final ppl_copy.
// Traffic: 3 * n * 2 bytes.

constexpr int kSwiThreads = 256;
constexpr int kSwiUnroll = 4;

template <bool IS_BF16>
TLM_DEV u32x4 swiglu8(u32x4 g, u32x4 u) {
  using H = h16<IS_BF16>;
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float g0 = H::lo(g[j]), g1 = H::hi(g[j]);
    float u0 = H::lo(u[j]), u1 = H::hi(u[j]);
    float s0 = g0 * __builtin_amdgcn_rcpf(fast_exp(-g0) + 1.0f);
    float s1 = g1 * __builtin_amdgcn_rcpf(fast_exp(-g1) + 1.0f);
    o[j] = H::pack(u0 * s0, u1 * s1);
  }
  return o;
}

// Each block streams contiguous chunks of kSwiThreads*kSwiUnroll vectors (all loads of a chunk
// issued before any math), grid-striding over chunks; this ordering measured faster than a
// whole-grid stride on MI355X.
template <bool IS_BF16>
__global__ __launch_bounds__(kSwiThreads) void swiglu_vec(const u32x4* __restrict__ gate,
                                                          const u32x4* __restrict__ up,
                                                          u32x4* __restrict__ out, int64_t nvec) {
  constexpr int64_t chunk = (int64_t)kSwiThreads * kSwiUnroll;
  for (int64_t c0 = (int64_t)blockIdx.x * chunk; c0 < nvec; c0 += (int64_t)gridDim.x * chunk) {
    u32x4 g[kSwiUnroll], u[kSwiUnroll];
#pragma unroll
    for (int k = 0; k < kSwiUnroll; ++k) {
      const int64_t i = c0 + k * kSwiThreads + threadIdx.x;
      if (i < nvec) {
        g[k] = ld_nt(gate + i);
        u[k] = ld_nt(up + i);
      }
    }
#pragma unroll
    for (int k = 0; k < kSwiUnroll; ++k) {
      const int64_t i = c0 + k * kSwiThreads + threadIdx.x;
      if (i < nvec) st_nt(out + i, swiglu8<IS_BF16>(g[k], u[k]));
    }
  }
}

template <bool IS_BF16>
__global__ __launch_bounds__(kSwiThreads) void swiglu_scalar(const uint16_t* __restrict__ gate,
                                                             const uint16_t* __restrict__ up,
                                                             uint16_t* __restrict__ out,
                                                             int64_t n) {
  using H = h16<IS_BF16>;
  for (int64_t i = (int64_t)blockIdx.x * kSwiThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kSwiThreads) {
    float g = H::to_f32(gate[i]), u = H::to_f32(up[i]);
    out[i] = (uint16_t)H::from_f32(u * (g * __builtin_amdgcn_rcpf(fast_exp(-g) + 1.0f)));
  }
}

// ------------------------------------------------------------------------------------------------
// RoPE. Reference program tpu_demo/tpu_test_rope_bf16.py:5-51 built on ppl_rope_add
// (codegen_ppl.cc:1809-1848): with x_cos = x*cos, x_sin = x*sin, x_neg_sin = -x*sin,
//   out[2i]   = x_cos[2i]   + x_neg_sin[2i+1] = x[2i]*cos[2i]     - x[2i+1]*sin[2i+1]
//   out[2i+1] = x_cos[2i+1] + x_sin[2i]       = x[2i+1]*cos[2i+1] + x[2i]*sin[2i]
// evaluated here in fp32 with one rounding. With the interleaved-duplicated tables of
// make_rope_cos_sin (:53-74) this equals rope_ref_torch (:76-92).
//
// Rows are (token, head) pairs of q then k: row r of the block's range belongs to token
// r / (Hq+Hk). A row of D elements is covered by D/8 lanes (16 bytes each); a lane reloads its
// table vector only when its token changes, so tables cost ~1 read per token.

constexpr int kRopeThreads = 256;
constexpr int kRopeRowsPerThread = 2;

template <bool IS_BF16, int LPR>
__global__ __launch_bounds__(kRopeThreads) void rope_vec(
    const u32x4* __restrict__ q, const u32x4* __restrict__ k, const u32x4* __restrict__ cos_t,
    const u32x4* __restrict__ sin_t, u32x4* __restrict__ q_out, u32x4* __restrict__ k_out,
    int64_t tokens, int hq, int hk) {
  using H = h16<IS_BF16>;
  constexpr int RPP = kRopeThreads / LPR;  // rows per pass
  const int htot = hq + hk;
  const int64_t nrows = tokens * htot;
  const int sub = threadIdx.x % LPR;
  const int64_t row0 = (int64_t)blockIdx.x * RPP * kRopeRowsPerThread + threadIdx.x / LPR;
  int64_t cur_tok = -1;
  u32x4 c = {0, 0, 0, 0}, s = {0, 0, 0, 0};
  u32x4 xs[kRopeRowsPerThread];
#pragma unroll
  for (int it = 0; it < kRopeRowsPerThread; ++it) {  // all row loads in flight first
    const int64_t row = row0 + (int64_t)it * RPP;
    if (row < nrows) {
      const int64_t t = row / htot;
      const int h = (int)(row - t * htot);
      xs[it] = ld_nt(h < hq ? q + (t * hq + h) * LPR + sub : k + (t * hk + (h - hq)) * LPR + sub);
    }
  }
#pragma unroll
  for (int it = 0; it < kRopeRowsPerThread; ++it) {
    const int64_t row = row0 + (int64_t)it * RPP;
    if (row >= nrows) break;
    const int64_t t = row / htot;
    const int h = (int)(row - t * htot);
    if (t != cur_tok) {
      c = cos_t[t * LPR + sub];
      s = sin_t[t * LPR + sub];
      cur_tok = t;
    }
    u32x4* dst = h < hq ? q_out + (t * hq + h) * LPR + sub : k_out + (t * hk + (h - hq)) * LPR + sub;
    const u32x4 x = xs[it];
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float xe = H::lo(x[j]), xo = H::hi(x[j]);
      const float ce = H::lo(c[j]), co = H::hi(c[j]);
      const float se = H::lo(s[j]), so = H::hi(s[j]);
      o[j] = H::pack(fmaf(xe, ce, -(xo * so)), fmaf(xo, co, xe * se));
    }
    st_nt(dst, o);
  }
}

// Any even D: one thread per (row, pair).
template <bool IS_BF16>
__global__ __launch_bounds__(kRopeThreads) void rope_scalar(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ cos_t, const uint16_t* __restrict__ sin_t,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out, int64_t tokens, int hq, int hk,
    int dim) {
  using H = h16<IS_BF16>;
  const int htot = hq + hk, half = dim / 2;
  const int64_t total = tokens * htot * half;
  for (int64_t i = (int64_t)blockIdx.x * kRopeThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kRopeThreads) {
    const int p = (int)(i % half);
    const int64_t row = i / half;
    const int64_t t = row / htot;
    const int h = (int)(row - t * htot);
    const uint16_t* src = h < hq ? q + (t * hq + h) * dim : k + (t * hk + (h - hq)) * dim;
    uint16_t* dst = h < hq ? q_out + (t * hq + h) * dim : k_out + (t * hk + (h - hq)) * dim;
    const uint16_t* ct = cos_t + t * dim;
    const uint16_t* st = sin_t + t * dim;
    const float xe = H::to_f32(src[2 * p]), xo = H::to_f32(src[2 * p + 1]);
    dst[2 * p] = (uint16_t)H::from_f32(fmaf(xe, H::to_f32(ct[2 * p]), -(xo * H::to_f32(st[2 * p + 1]))));
    dst[2 * p + 1] = (uint16_t)H::from_f32(fmaf(xo, H::to_f32(ct[2 * p + 1]), xe * H::to_f32(st[2 * p])));
  }
}

unsigned grid_for(int64_t work, int per_block, int64_t cap) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g > cap) g = cap;
  return (unsigned)(g < 1 ? 1 : g);
}

template <bool IS_BF16, int LPR>
void launch_rope_vec(const void* q, const void* k, const void* c, const void* s, void* qo,
                     void* ko, int64_t tokens, int hq, int hk, hipStream_t st) {
  constexpr int RPP = kRopeThreads / LPR;
  const int64_t nrows = tokens * (hq + hk);
  unsigned grid = grid_for(nrows, RPP * kRopeRowsPerThread, INT32_MAX);
  rope_vec<IS_BF16, LPR><<<grid, kRopeThreads, 0, st>>>(
      (const u32x4*)q, (const u32x4*)k, (const u32x4*)c, (const u32x4*)s, (u32x4*)qo,
      (u32x4*)ko, tokens, hq, hk);
}

template <bool IS_BF16>
int rope_dispatch(const void* q, const void* k, const void* c, const void* s, void* qo, void* ko,
                  int64_t tokens, int hq, int hk, int dim, hipStream_t st) {
  bool vec = tlm_aligned(q, 16) && tlm_aligned(qo, 16) && tlm_aligned(c, 16) &&
             tlm_aligned(s, 16) && (!k || (tlm_aligned(k, 16) && tlm_aligned(ko, 16)));
  if (vec && dim == 128)
    launch_rope_vec<IS_BF16, 16>(q, k, c, s, qo, ko, tokens, hq, hk, st);
  else if (vec && dim == 64)
    launch_rope_vec<IS_BF16, 8>(q, k, c, s, qo, ko, tokens, hq, hk, st);
  else if (vec && dim == 256)
    launch_rope_vec<IS_BF16, 32>(q, k, c, s, qo, ko, tokens, hq, hk, st);
  else {
    int64_t total = tokens * (hq + hk) * (dim / 2);
    rope_scalar<IS_BF16><<<grid_for(total, kRopeThreads, 1 << 20), kRopeThreads, 0, st>>>(
        (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)c, (const uint16_t*)s,
        (uint16_t*)qo, (uint16_t*)ko, tokens, hq, hk, dim);
  }
  TLM_LAUNCH_CHECK("tlm_rope");
  return TLM_OK;
}

}  // namespace

extern "C" int tlm_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype,
                          void* stream) {
  if (!gate || !up || !out) {
    tlm_set_error("tlm_swiglu: null pointer");
    return TLM_EINVAL;
  }
  if (n < 0) {
    tlm_set_error("tlm_swiglu: negative size");
    return TLM_EINVAL;
  }
  if (!tlm_aligned(gate, 2) || !tlm_aligned(up, 2) || !tlm_aligned(out, 2)) {
    tlm_set_error("tlm_swiglu: pointers must be 2-byte aligned");
    return TLM_EINVAL;
  }
  if (dtype != TLM_F16 && dtype != TLM_BF16) {
    tlm_set_error("tlm_swiglu: dtype %d unsupported (F16 or BF16)", dtype);
    return TLM_EUNSUPPORTED;
  }
  if (n == 0) return TLM_OK;
  hipStream_t s = (hipStream_t)stream;
  const bool bf = dtype == TLM_BF16;
  if (n % 8 == 0 && tlm_aligned(gate, 16) && tlm_aligned(up, 16) && tlm_aligned(out, 16)) {
    const int64_t nvec = n / 8;
    // 1024 blocks (4 per CU) streaming 16 KiB chunks measured best at the 8192x14336 config.
    unsigned grid = grid_for(nvec, kSwiThreads * kSwiUnroll, 1024);
    if (bf)
      swiglu_vec<true><<<grid, kSwiThreads, 0, s>>>((const u32x4*)gate, (const u32x4*)up,
                                                     (u32x4*)out, nvec);
    else
      swiglu_vec<false><<<grid, kSwiThreads, 0, s>>>((const u32x4*)gate, (const u32x4*)up,
                                                      (u32x4*)out, nvec);
  } else {
    unsigned grid = grid_for(n, kSwiThreads, 256 * 16);
    if (bf)
      swiglu_scalar<true><<<grid, kSwiThreads, 0, s>>>((const uint16_t*)gate,
                                                        (const uint16_t*)up, (uint16_t*)out, n);
    else
      swiglu_scalar<false><<<grid, kSwiThreads, 0, s>>>((const uint16_t*)gate,
                                                         (const uint16_t*)up, (uint16_t*)out, n);
  }
  TLM_LAUNCH_CHECK("tlm_swiglu");
  return TLM_OK;
}

extern "C" int tlm_rope(const void* q, const void* k, const void* cos_t, const void* sin_t,
                        void* q_out, void* k_out, int64_t tokens, int64_t heads_q, int64_t heads_k,
                        int64_t dim, int dtype, void* stream) {
  if (!q || !cos_t || !sin_t || !q_out) {
    tlm_set_error("tlm_rope: null q, cos, sin or q_out");
    return TLM_EINVAL;
  }
  if ((k == nullptr) != (k_out == nullptr)) {
    tlm_set_error("tlm_rope: k and k_out must both be given or both be NULL");
    return TLM_EINVAL;
  }
  if (!k) heads_k = 0;
  if (tokens < 0 || heads_q <= 0 || heads_k < 0 || dim <= 0 || dim % 2 != 0 ||
      heads_q + heads_k > (1 << 20) || dim > (1 << 20)) {
    tlm_set_error("tlm_rope: bad shape tokens=%lld heads_q=%lld heads_k=%lld dim=%lld (dim even)",
                  (long long)tokens, (long long)heads_q, (long long)heads_k, (long long)dim);
    return TLM_EINVAL;
  }
  if (!tlm_aligned(q, 2) || !tlm_aligned(cos_t, 2) || !tlm_aligned(sin_t, 2) ||
      !tlm_aligned(q_out, 2) || (k && (!tlm_aligned(k, 2) || !tlm_aligned(k_out, 2)))) {
    tlm_set_error("tlm_rope: pointers must be 2-byte aligned");
    return TLM_EINVAL;
  }
  if (dtype != TLM_F16 && dtype != TLM_BF16) {
    tlm_set_error("tlm_rope: dtype %d unsupported (F16 or BF16)", dtype);
    return TLM_EUNSUPPORTED;
  }
  if (tokens == 0) return TLM_OK;
  hipStream_t s = (hipStream_t)stream;
  return dtype == TLM_BF16
             ? rope_dispatch<true>(q, k, cos_t, sin_t, q_out, k_out, tokens, (int)heads_q,
                                   (int)heads_k, (int)dim, s)
             : rope_dispatch<false>(q, k, cos_t, sin_t, q_out, k_out, tokens, (int)heads_q,
                                    (int)heads_k, (int)dim, s);
}
