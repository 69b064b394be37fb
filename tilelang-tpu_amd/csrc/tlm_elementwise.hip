// HBM-streaming elementwise kernels: SwiGLU and interleaved RoPE.
// No MFMA and no LDS: every byte is read once with 16-byte vector loads, math in fp32, one
// rounding per output, 16-byte stores (cache policies per kernel below).
#include "tlm_common.h"

#include <algorithm>

namespace {

// ------------------------------------------------------------------------------------------------
// SwiGLU. Reference program tpu_demo/tpu_test_swiglu_bf16.py:5-54:
//   x = fp32(gate); e = exp(-x) (ppl_exp2 = natural exp, codegen_ppl.cc:1294-1320);
//   out = cast(up * (x / (e + 1)))   — fp32 throughout, one rounding at the final ppl_copy.
// Traffic: 3 * n * 2 bytes.

constexpr int kSwiThreads = 256;
constexpr int kSwiUnroll = 4;    // fp32 kernel: 16-byte vectors per thread and chunk
constexpr int kSwiUnroll16 = 2;  // 16-bit kernel: 16-byte vectors per thread and chunk
// Cache policies (st_cp / ld_cp): non-temporal loads, stores with sc0 sc1 (system scope,
// written through). Measured on the config (8192 x 14336 bf16, back to back): 6.73-6.76 TB/s
// against 6.26 TB/s with non-temporal stores and four vectors per thread.
constexpr int kSwiLoadCP = CP_GLOBAL_NT, kSwiStoreCP = CP_SC01;

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
  constexpr int64_t chunk = (int64_t)kSwiThreads * kSwiUnroll16;
  for (int64_t c0 = (int64_t)blockIdx.x * chunk; c0 < nvec; c0 += (int64_t)gridDim.x * chunk) {
    u32x4 g[kSwiUnroll16], u[kSwiUnroll16];
    const u32x4* gb = gate + c0;  // chunk bases: uniform over the workgroup
    const u32x4* ub = up + c0;
    u32x4* ob = out + c0;
#pragma unroll
    for (int k = 0; k < kSwiUnroll16; ++k) {
      const int j = k * kSwiThreads + (int)threadIdx.x;
      if (c0 + j < nvec) {
        g[k] = ld_cp<kSwiLoadCP>(gb, j * 16);
        u[k] = ld_cp<kSwiLoadCP>(ub, j * 16);
      }
    }
#pragma unroll
    for (int k = 0; k < kSwiUnroll16; ++k) {
      const int j = k * kSwiThreads + (int)threadIdx.x;
      if (c0 + j < nvec) st_cp<kSwiStoreCP>(ob, j * 16, swiglu8<IS_BF16>(g[k], u[k]));
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
// Cache policies of rope_tok's row loads and output stores (st_cp / ld_cp): non-temporal loads,
// stores with sc0 sc1. Measured on the config (q, k [8192, 32, 128] bf16, back to back): 6.76-6.77
// TB/s against 6.24 TB/s with non-temporal stores.
constexpr int kRopeLoadCP = CP_GLOBAL_NT, kRopeStoreCP = CP_SC01;

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

// One token per workgroup iteration: the token's cos / sin vector is loaded once per lane and
// applied to all its q and k heads (LPR lanes per head row, 256 / LPR rows in flight per pass,
// four passes' loads issued before any store).
template <bool IS_BF16, int LPR>
__global__ __launch_bounds__(kRopeThreads) void rope_tok(
    const u32x4* __restrict__ q, const u32x4* __restrict__ k, const u32x4* __restrict__ cos_t,
    const u32x4* __restrict__ sin_t, u32x4* __restrict__ q_out, u32x4* __restrict__ k_out,
    int64_t tokens, int hq, int hk) {
  using H = h16<IS_BF16>;
  constexpr int SLOTS = kRopeThreads / LPR;  // head rows per pass
  constexpr int U = 4;                        // passes in flight
  const int htot = hq + hk;
  const int sub = threadIdx.x % LPR, slot = threadIdx.x / LPR;
  for (int64_t t = blockIdx.x; t < tokens; t += gridDim.x) {
    const u32x4 c = cos_t[t * LPR + sub], s = sin_t[t * LPR + sub];
    // the token's q and k rows: bases uniform over the workgroup, lane offsets in bytes
    const u32x4* qt = q + t * hq * LPR;
    const u32x4* kt = k + t * hk * LPR;
    u32x4* qo = q_out + t * hq * LPR;
    u32x4* ko = k_out + t * hk * LPR;
    for (int h0 = slot; h0 < htot; h0 += U * SLOTS) {
      u32x4 xs[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int h = h0 + u * SLOTS;
        if (h < htot)
          xs[u] = h < hq ? ld_cp<kRopeLoadCP>(qt, (h * LPR + sub) * 16)
                         : ld_cp<kRopeLoadCP>(kt, ((h - hq) * LPR + sub) * 16);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int h = h0 + u * SLOTS;
        if (h >= htot) break;
        const u32x4 x = xs[u];
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float xe = H::lo(x[j]), xo = H::hi(x[j]);
          const float ce = H::lo(c[j]), co = H::hi(c[j]);
          const float se = H::lo(s[j]), so = H::hi(s[j]);
          o[j] = H::pack(fmaf(xe, ce, -(xo * so)), fmaf(xo, co, xe * se));
        }
        if (h < hq)
          st_cp<kRopeStoreCP>(qo, (h * LPR + sub) * 16, o);
        else
          st_cp<kRopeStoreCP>(ko, ((h - hq) * LPR + sub) * 16, o);
      }
    }
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

// ------------------------------------------------------------------------------------------------
// fp32 programs (tpu_demo/tpu_test_swiglu_fp32.py, tpu_test_rope_fp32.py, tpu_test_rope.py): the
// same expressions on fp32 tiles, stored as fp32 (no rounding step).

TLM_DEV float swiglu1(float g, float u) {
  return u * (g * __builtin_amdgcn_rcpf(fast_exp(-g) + 1.0f));
}

__global__ __launch_bounds__(kSwiThreads) void swiglu_f32_vec(const f32x4* __restrict__ gate,
                                                              const f32x4* __restrict__ up,
                                                              f32x4* __restrict__ out,
                                                              int64_t nvec) {
  constexpr int64_t chunk = (int64_t)kSwiThreads * kSwiUnroll;
  for (int64_t c0 = (int64_t)blockIdx.x * chunk; c0 < nvec; c0 += (int64_t)gridDim.x * chunk) {
    f32x4 g[kSwiUnroll], u[kSwiUnroll];
#pragma unroll
    for (int k = 0; k < kSwiUnroll; ++k) {
      const int64_t i = c0 + k * kSwiThreads + threadIdx.x;
      if (i < nvec) {
        g[k] = __builtin_nontemporal_load(gate + i);
        u[k] = __builtin_nontemporal_load(up + i);
      }
    }
#pragma unroll
    for (int k = 0; k < kSwiUnroll; ++k) {
      const int64_t i = c0 + k * kSwiThreads + threadIdx.x;
      if (i < nvec) {
        f32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = swiglu1(g[k][j], u[k][j]);
        __builtin_nontemporal_store(o, out + i);
      }
    }
  }
}

__global__ __launch_bounds__(kSwiThreads) void swiglu_f32_scalar(const float* __restrict__ gate,
                                                                 const float* __restrict__ up,
                                                                 float* __restrict__ out,
                                                                 int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kSwiThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kSwiThreads)
    out[i] = swiglu1(gate[i], up[i]);
}

// fp32 RoPE, dim % 4 == 0: one thread per 16-byte chunk (two pairs) of a (token, head) row.
__global__ __launch_bounds__(kRopeThreads) void rope_f32_vec(
    const f32x4* __restrict__ q, const f32x4* __restrict__ k, const f32x4* __restrict__ cos_t,
    const f32x4* __restrict__ sin_t, f32x4* __restrict__ q_out, f32x4* __restrict__ k_out,
    int64_t tokens, int hq, int hk, int cpr) {
  const int htot = hq + hk;
  const int64_t total = tokens * htot * cpr;
  for (int64_t i = (int64_t)blockIdx.x * kRopeThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kRopeThreads) {
    const int c = (int)(i % cpr);
    const int64_t row = i / cpr;
    const int64_t t = row / htot;
    const int h = (int)(row - t * htot);
    const int64_t off = (h < hq ? t * hq + h : t * hk + (h - hq)) * cpr + c;
    const f32x4 x = h < hq ? q[off] : k[off];
    const f32x4 cv = cos_t[t * cpr + c], sv = sin_t[t * cpr + c];
    f32x4 o;
#pragma unroll
    for (int j = 0; j < 4; j += 2) {
      o[j] = fmaf(x[j], cv[j], -(x[j + 1] * sv[j + 1]));
      o[j + 1] = fmaf(x[j + 1], cv[j + 1], x[j] * sv[j]);
    }
    if (h < hq)
      q_out[off] = o;
    else
      k_out[off] = o;
  }
}

// fp32 RoPE, any even dim: one thread per pair.
__global__ __launch_bounds__(kRopeThreads) void rope_f32_scalar(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, float* __restrict__ q_out, float* __restrict__ k_out,
    int64_t tokens, int hq, int hk, int dim) {
  const int htot = hq + hk, half = dim / 2;
  const int64_t total = tokens * htot * half;
  for (int64_t i = (int64_t)blockIdx.x * kRopeThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kRopeThreads) {
    const int p = (int)(i % half);
    const int64_t row = i / half;
    const int64_t t = row / htot;
    const int h = (int)(row - t * htot);
    const float* src = h < hq ? q + (t * hq + h) * dim : k + (t * hk + (h - hq)) * dim;
    float* dst = h < hq ? q_out + (t * hq + h) * dim : k_out + (t * hk + (h - hq)) * dim;
    const float* ct = cos_t + t * dim;
    const float* st = sin_t + t * dim;
    const float xe = src[2 * p], xo = src[2 * p + 1];
    dst[2 * p] = fmaf(xe, ct[2 * p], -(xo * st[2 * p + 1]));
    dst[2 * p + 1] = fmaf(xo, ct[2 * p + 1], xe * st[2 * p]);
  }
}

// ------------------------------------------------------------------------------------------------
// dtype conversion of a tile copy between global tensors (ppl_copy with differing dtypes,
// codegen_ppl.cc:1138-1152): fp32 -> fp16 / bf16 rounds to nearest even, 16-bit -> fp32 is exact.

template <int SRC, int DST>
TLM_DEV float cast_load(const void* p, int64_t i) {
  if constexpr (SRC == TLM_F32) return ((const float*)p)[i];
  else return h16<SRC == TLM_BF16>::to_f32(((const uint16_t*)p)[i]);
}

template <int SRC, int DST>
__global__ __launch_bounds__(256) void cast_scalar(const void* __restrict__ src,
                                                   void* __restrict__ dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256) {
    const float v = cast_load<SRC, DST>(src, i);
    if constexpr (DST == TLM_F32) ((float*)dst)[i] = v;
    else ((uint16_t*)dst)[i] = (uint16_t)h16<DST == TLM_BF16>::from_f32(v);
  }
}

// 8 elements per thread and iteration: 2 x 16 bytes of fp32 <-> 16 bytes of 16-bit values.
template <int SRC, int DST>
__global__ __launch_bounds__(256) void cast_vec8(const void* __restrict__ src,
                                                 void* __restrict__ dst, int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * 256) {
    if constexpr (SRC == TLM_F32) {
      const f32x4 a = ((const f32x4*)src)[2 * i], b = ((const f32x4*)src)[2 * i + 1];
      using H = h16<DST == TLM_BF16>;
      ((u32x4*)dst)[i] = u32x4{H::pack(a[0], a[1]), H::pack(a[2], a[3]), H::pack(b[0], b[1]),
                               H::pack(b[2], b[3])};
    } else {
      using H = h16<SRC == TLM_BF16>;
      const u32x4 w = ((const u32x4*)src)[i];
      ((f32x4*)dst)[2 * i] = f32x4{H::lo(w[0]), H::hi(w[0]), H::lo(w[1]), H::hi(w[1])};
      ((f32x4*)dst)[2 * i + 1] = f32x4{H::lo(w[2]), H::hi(w[2]), H::lo(w[3]), H::hi(w[3])};
    }
  }
}

template <int SRC, int DST>
void launch_cast(const void* src, void* dst, int64_t n, hipStream_t st);

unsigned grid_for(int64_t work, int per_block, int64_t cap) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g > cap) g = cap;
  return (unsigned)(g < 1 ? 1 : g);
}

template <bool IS_BF16, int LPR>
void launch_rope_vec(const void* q, const void* k, const void* c, const void* s, void* qo,
                     void* ko, int64_t tokens, int hq, int hk, hipStream_t st) {
  constexpr int RPP = kRopeThreads / LPR;
  if (hq + hk >= RPP) {  // a token fills at least one pass: one token per workgroup iteration
    rope_tok<IS_BF16, LPR><<<(unsigned)std::min<int64_t>(tokens, 1 << 20), kRopeThreads, 0,
                             st>>>((const u32x4*)q, (const u32x4*)k, (const u32x4*)c,
                                   (const u32x4*)s, (u32x4*)qo, (u32x4*)ko, tokens, hq, hk);
    return;
  }
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

template <int SRC, int DST>
void launch_cast(const void* src, void* dst, int64_t n, hipStream_t st) {
  if (n % 8 == 0 && tlm_aligned(src, 16) && tlm_aligned(dst, 16))
    cast_vec8<SRC, DST><<<grid_for(n / 8, 256, 256 * 16), 256, 0, st>>>(src, dst, n / 8);
  else
    cast_scalar<SRC, DST><<<grid_for(n, 256, 256 * 16), 256, 0, st>>>(src, dst, n);
}

}  // namespace

extern "C" int tlm_cast(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n,
                        void* stream) {
  if (!src || !dst) {
    tlm_set_error("tlm_cast: null pointer");
    return TLM_EINVAL;
  }
  if (n < 0) {
    tlm_set_error("tlm_cast: negative size");
    return TLM_EINVAL;
  }
  const bool f32_to_16 = src_dtype == TLM_F32 && (dst_dtype == TLM_F16 || dst_dtype == TLM_BF16);
  const bool h16_to_f32 = dst_dtype == TLM_F32 && (src_dtype == TLM_F16 || src_dtype == TLM_BF16);
  if (!f32_to_16 && !h16_to_f32) {
    tlm_set_error("tlm_cast: %d -> %d unsupported (F32 <-> F16 / BF16)", src_dtype, dst_dtype);
    return TLM_EUNSUPPORTED;
  }
  if (!tlm_aligned(src, src_dtype == TLM_F32 ? 4 : 2) ||
      !tlm_aligned(dst, dst_dtype == TLM_F32 ? 4 : 2)) {
    tlm_set_error("tlm_cast: pointers must be aligned to their element size");
    return TLM_EINVAL;
  }
  if (n == 0) return TLM_OK;
  hipStream_t st = (hipStream_t)stream;
  if (f32_to_16) {
    if (dst_dtype == TLM_F16) launch_cast<TLM_F32, TLM_F16>(src, dst, n, st);
    else launch_cast<TLM_F32, TLM_BF16>(src, dst, n, st);
  } else {
    if (src_dtype == TLM_F16) launch_cast<TLM_F16, TLM_F32>(src, dst, n, st);
    else launch_cast<TLM_BF16, TLM_F32>(src, dst, n, st);
  }
  TLM_LAUNCH_CHECK("tlm_cast");
  return TLM_OK;
}

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
  if (dtype != TLM_F16 && dtype != TLM_BF16 && dtype != TLM_F32) {
    tlm_set_error("tlm_swiglu: dtype %d unsupported (F16, BF16 or F32)", dtype);
    return TLM_EUNSUPPORTED;
  }
  const int esz = dtype == TLM_F32 ? 4 : 2;
  if (!tlm_aligned(gate, esz) || !tlm_aligned(up, esz) || !tlm_aligned(out, esz)) {
    tlm_set_error("tlm_swiglu: pointers must be aligned to the element size");
    return TLM_EINVAL;
  }
  if (n == 0) return TLM_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TLM_F32) {
    if (n % 4 == 0 && tlm_aligned(gate, 16) && tlm_aligned(up, 16) && tlm_aligned(out, 16))
      swiglu_f32_vec<<<grid_for(n / 4, kSwiThreads * kSwiUnroll, 1024), kSwiThreads, 0, s>>>(
          (const f32x4*)gate, (const f32x4*)up, (f32x4*)out, n / 4);
    else
      swiglu_f32_scalar<<<grid_for(n, kSwiThreads, 256 * 16), kSwiThreads, 0, s>>>(
          (const float*)gate, (const float*)up, (float*)out, n);
    TLM_LAUNCH_CHECK("tlm_swiglu");
    return TLM_OK;
  }
  const bool bf = dtype == TLM_BF16;
  if (n % 8 == 0 && tlm_aligned(gate, 16) && tlm_aligned(up, 16) && tlm_aligned(out, 16)) {
    const int64_t nvec = n / 8;
    // 1024 blocks (4 per CU) streaming 16 KiB chunks measured best at the 8192x14336 config.
    unsigned grid = grid_for(nvec, kSwiThreads * kSwiUnroll16, 1024);
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
  if (dtype != TLM_F16 && dtype != TLM_BF16 && dtype != TLM_F32) {
    tlm_set_error("tlm_rope: dtype %d unsupported (F16, BF16 or F32)", dtype);
    return TLM_EUNSUPPORTED;
  }
  const int esz = dtype == TLM_F32 ? 4 : 2;
  if (!tlm_aligned(q, esz) || !tlm_aligned(cos_t, esz) || !tlm_aligned(sin_t, esz) ||
      !tlm_aligned(q_out, esz) || (k && (!tlm_aligned(k, esz) || !tlm_aligned(k_out, esz)))) {
    tlm_set_error("tlm_rope: pointers must be aligned to the element size");
    return TLM_EINVAL;
  }
  if (tokens == 0) return TLM_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TLM_F32) {
    const bool vec = dim % 4 == 0 && tlm_aligned(q, 16) && tlm_aligned(q_out, 16) &&
                     tlm_aligned(cos_t, 16) && tlm_aligned(sin_t, 16) &&
                     (!k || (tlm_aligned(k, 16) && tlm_aligned(k_out, 16)));
    if (vec) {
      const int64_t total = tokens * (heads_q + heads_k) * (dim / 4);
      rope_f32_vec<<<grid_for(total, kRopeThreads, 1 << 20), kRopeThreads, 0, s>>>(
          (const f32x4*)q, (const f32x4*)k, (const f32x4*)cos_t, (const f32x4*)sin_t,
          (f32x4*)q_out, (f32x4*)k_out, tokens, (int)heads_q, (int)heads_k, (int)(dim / 4));
    } else {
      const int64_t total = tokens * (heads_q + heads_k) * (dim / 2);
      rope_f32_scalar<<<grid_for(total, kRopeThreads, 1 << 20), kRopeThreads, 0, s>>>(
          (const float*)q, (const float*)k, (const float*)cos_t, (const float*)sin_t,
          (float*)q_out, (float*)k_out, tokens, (int)heads_q, (int)heads_k, (int)dim);
    }
    TLM_LAUNCH_CHECK("tlm_rope");
    return TLM_OK;
  }
  return dtype == TLM_BF16
             ? rope_dispatch<true>(q, k, cos_t, sin_t, q_out, k_out, tokens, (int)heads_q,
                                   (int)heads_k, (int)dim, s)
             : rope_dispatch<false>(q, k, cos_t, sin_t, q_out, k_out, tokens, (int)heads_q,
                                    (int)heads_k, (int)dim, s);
}
