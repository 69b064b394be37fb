// RMSNorm forward, one row per 64-lane wavefront, single pass over HBM.
//
// Reference program: tpu_demo/rms_norm/rms_norm_fp16.py:9-35 — per row, fp32 compute:
//   x32 = fp32(x); s = sum(x32*x32) (ppl_reduce_sum, codegen_ppl.cc:1554-1792);
//   s = s * (1/N) + eps; r = rsqrt(s) (ppl_rsqrt); y = cast(x32 * r)   (ppl_copy with cast, RNE).
// The optional weight w (fp16/bf16 [cols]) is applied in fp32 before the single rounding.
//
// fp32 programs (tpu_demo/rms_norm/rmsnorm_fp32.py, rmsnorm_splitk_fp32.py) compute the same
// expression on fp32 tiles and store fp32 (no rounding step); the split-K programs
// (rmsnorm_splitk_fp16.py:9-47) accumulate the same row sum over column blocks, so they map to
// the same kernels.
//
// Layout: x, y [rows, cols] row-major 16-bit or fp32. Each lane keeps its slice of the row in
// VGPRs (cols/512 or cols/256 16-byte vectors per lane), so x is read exactly once and y written
// once: algorithmic traffic = 2*rows*cols*esize + cols*esize bytes. No MFMA: the sum of squares reduces with
// xor-shuffles across the wavefront.
#include "tlm_common.h"

namespace {

constexpr int kWavesPerBlock = 4;
// Cache policies of the row loads and the output stores (st_cp / ld_cp): plain loads and
// non-temporal stores. Stores with sc0 sc1, which speed up the SwiGLU and RoPE streams, measured
// slower here back to back (5.0 against 6.1 TB/s at 4096^2).
constexpr int kRmsLoadCP = CP_GLOBAL, kRmsStoreCP = CP_NT;
constexpr bool kRmsWeightFirst = false;  // weight loads issued with the row's (ahead of the sum)

// VPL = 16-byte vectors per lane; the row has exactly 64*VPL*8 elements (cols == 512*VPL).
template <bool IS_BF16, int VPL, bool HAS_W>
__global__ __launch_bounds__(64 * kWavesPerBlock) void rmsnorm_row_regs(
    const u32x4* __restrict__ x, const u32x4* __restrict__ w, u32x4* __restrict__ y,
    int64_t rows, float inv_cols, float eps) {
  using H = h16<IS_BF16>;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock +
                      __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  if (row >= rows) return;
  const u32x4* xr = x + row * (64 * VPL);
  u32x4* yr = y + row * (64 * VPL);

  u32x4 v[VPL], wv[HAS_W && kRmsWeightFirst ? VPL : 1];
#pragma unroll
  for (int i = 0; i < VPL; ++i) v[i] = ld_cp<kRmsLoadCP>(xr, (i * 64 + lane) * 16);
  if constexpr (HAS_W && kRmsWeightFirst) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) wv[i] = w[i * 64 + lane];
  }

  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float a = H::lo(v[i][j]), b = H::hi(v[i][j]);
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
  ss = wave_sum(ss);
  const float r = __frsqrt_rn(ss * inv_cols + eps);

#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    u32x4 o;
    if constexpr (HAS_W) {
      const u32x4 wi = kRmsWeightFirst ? wv[HAS_W && kRmsWeightFirst ? i : 0] : w[i * 64 + lane];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = H::pack(H::lo(v[i][j]) * r * H::lo(wi[j]), H::hi(v[i][j]) * r * H::hi(wi[j]));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = H::pack(H::lo(v[i][j]) * r, H::hi(v[i][j]) * r);
    }
    st_cp<kRmsStoreCP>(yr, (i * 64 + lane) * 16, o);
  }
}

// Any shape: two passes over the row (sum, then scale), scalar 16-bit accesses.
template <bool IS_BF16>
__global__ __launch_bounds__(64 * kWavesPerBlock) void rmsnorm_row_generic(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
    int64_t rows, int64_t cols, float inv_cols, float eps) {
  using H = h16<IS_BF16>;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* xr = x + row * cols;
  uint16_t* yr = y + row * cols;
  float ss = 0.f;
  for (int64_t c = lane; c < cols; c += 64) {
    float a = H::to_f32(xr[c]);
    ss = fmaf(a, a, ss);
  }
  ss = wave_sum(ss);
  const float r = __frsqrt_rn(ss * inv_cols + eps);
  for (int64_t c = lane; c < cols; c += 64) {
    float a = H::to_f32(xr[c]) * r;
    if (w) a *= H::to_f32(w[c]);
    yr[c] = (uint16_t)H::from_f32(a);
  }
}

// fp32 rows: VPL 16-byte vectors (4 floats) per lane, cols == 256*VPL; row kept in VGPRs.
template <int VPL, bool HAS_W>
__global__ __launch_bounds__(64 * kWavesPerBlock) void rmsnorm_f32_regs(
    const f32x4* __restrict__ x, const f32x4* __restrict__ w, f32x4* __restrict__ y,
    int64_t rows, float inv_cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const f32x4* xr = x + row * (64 * VPL);
  f32x4* yr = y + row * (64 * VPL);
  f32x4 v[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) v[i] = xr[i * 64 + lane];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) ss = fmaf(v[i][j], v[i][j], ss);
  ss = wave_sum(ss);
  const float r = __frsqrt_rn(ss * inv_cols + eps);
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    f32x4 o;
    if constexpr (HAS_W) {
      const f32x4 wv = w[i * 64 + lane];
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = v[i][j] * r * wv[j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = v[i][j] * r;
    }
    __builtin_nontemporal_store(o, yr + i * 64 + lane);
  }
}

__global__ __launch_bounds__(64 * kWavesPerBlock) void rmsnorm_f32_generic(
    const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y, int64_t rows,
    int64_t cols, float inv_cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + row * cols;
  float* yr = y + row * cols;
  float ss = 0.f;
  for (int64_t c = lane; c < cols; c += 64) ss = fmaf(xr[c], xr[c], ss);
  ss = wave_sum(ss);
  const float r = __frsqrt_rn(ss * inv_cols + eps);
  for (int64_t c = lane; c < cols; c += 64) yr[c] = w ? xr[c] * r * w[c] : xr[c] * r;
}

template <int VPL>
void launch_f32_regs(const void* x, const void* w, void* y, int64_t rows, float inv, float eps,
                     hipStream_t s, dim3 grid, dim3 block) {
  if (w)
    rmsnorm_f32_regs<VPL, true><<<grid, block, 0, s>>>((const f32x4*)x, (const f32x4*)w,
                                                       (f32x4*)y, rows, inv, eps);
  else
    rmsnorm_f32_regs<VPL, false><<<grid, block, 0, s>>>((const f32x4*)x, nullptr, (f32x4*)y,
                                                        rows, inv, eps);
}

int dispatch_f32(const void* x, const void* w, void* y, int64_t rows, int64_t cols, float eps,
                 hipStream_t s) {
  const float inv = 1.0f / (float)cols;
  dim3 block(64 * kWavesPerBlock);
  dim3 grid((unsigned)((rows + kWavesPerBlock - 1) / kWavesPerBlock));
  const bool vec_ok = tlm_aligned(x, 16) && tlm_aligned(y, 16) && (!w || tlm_aligned(w, 16));
  const int64_t vpl = cols / 256;
  if (vec_ok && cols % 256 == 0 && (vpl == 1 || vpl == 2 || vpl == 4 || vpl == 8 || vpl == 16)) {
    switch (vpl) {
      case 1: launch_f32_regs<1>(x, w, y, rows, inv, eps, s, grid, block); break;
      case 2: launch_f32_regs<2>(x, w, y, rows, inv, eps, s, grid, block); break;
      case 4: launch_f32_regs<4>(x, w, y, rows, inv, eps, s, grid, block); break;
      case 8: launch_f32_regs<8>(x, w, y, rows, inv, eps, s, grid, block); break;
      default: launch_f32_regs<16>(x, w, y, rows, inv, eps, s, grid, block); break;
    }
  } else {
    rmsnorm_f32_generic<<<grid, block, 0, s>>>((const float*)x, (const float*)w, (float*)y, rows,
                                               cols, inv, eps);
  }
  TLM_LAUNCH_CHECK("tlm_rmsnorm");
  return TLM_OK;
}

template <bool IS_BF16, int VPL>
void launch_regs(const void* x, const void* w, void* y, int64_t rows, float inv, float eps,
                 hipStream_t s, dim3 grid, dim3 block) {
  if (w)
    rmsnorm_row_regs<IS_BF16, VPL, true><<<grid, block, 0, s>>>(
        (const u32x4*)x, (const u32x4*)w, (u32x4*)y, rows, inv, eps);
  else
    rmsnorm_row_regs<IS_BF16, VPL, false><<<grid, block, 0, s>>>(
        (const u32x4*)x, nullptr, (u32x4*)y, rows, inv, eps);
}

template <bool IS_BF16>
int dispatch(const void* x, const void* w, void* y, int64_t rows, int64_t cols, float eps,
             hipStream_t s) {
  const float inv = 1.0f / (float)cols;
  dim3 block(64 * kWavesPerBlock);
  dim3 grid((unsigned)((rows + kWavesPerBlock - 1) / kWavesPerBlock));
  const bool vec_ok = tlm_aligned(x, 16) && tlm_aligned(y, 16) && (!w || tlm_aligned(w, 16));
  if (vec_ok && cols % 512 == 0 && cols / 512 <= 16) {
    switch (cols / 512) {
      case 1: launch_regs<IS_BF16, 1>(x, w, y, rows, inv, eps, s, grid, block); break;
      case 2: launch_regs<IS_BF16, 2>(x, w, y, rows, inv, eps, s, grid, block); break;
      case 4: launch_regs<IS_BF16, 4>(x, w, y, rows, inv, eps, s, grid, block); break;
      case 8: launch_regs<IS_BF16, 8>(x, w, y, rows, inv, eps, s, grid, block); break;
      case 16: launch_regs<IS_BF16, 16>(x, w, y, rows, inv, eps, s, grid, block); break;
      default:
        rmsnorm_row_generic<IS_BF16><<<grid, block, 0, s>>>(
            (const uint16_t*)x, (const uint16_t*)w, (uint16_t*)y, rows, cols, inv, eps);
    }
  } else {
    rmsnorm_row_generic<IS_BF16><<<grid, block, 0, s>>>(
        (const uint16_t*)x, (const uint16_t*)w, (uint16_t*)y, rows, cols, inv, eps);
  }
  TLM_LAUNCH_CHECK("tlm_rmsnorm");
  return TLM_OK;
}

}  // namespace

extern "C" int tlm_rmsnorm(const void* x, const void* w, void* y, int64_t rows, int64_t cols,
                           float eps, int dtype, void* stream) {
  if (!x || !y) {
    tlm_set_error("tlm_rmsnorm: null x or y");
    return TLM_EINVAL;
  }
  if (rows < 0 || cols <= 0 || rows > (int64_t)0xffffffff * kWavesPerBlock) {
    tlm_set_error("tlm_rmsnorm: bad shape rows=%lld cols=%lld", (long long)rows, (long long)cols);
    return TLM_EINVAL;
  }
  const int esz = dtype == TLM_F32 ? 4 : 2;
  if (!tlm_aligned(x, esz) || !tlm_aligned(y, esz) || (w && !tlm_aligned(w, esz))) {
    tlm_set_error("tlm_rmsnorm: pointers must be aligned to the element size");
    return TLM_EINVAL;
  }
  if (!(eps >= 0.f)) {
    tlm_set_error("tlm_rmsnorm: eps must be >= 0");
    return TLM_EINVAL;
  }
  if (dtype != TLM_F16 && dtype != TLM_BF16 && dtype != TLM_F32) {
    tlm_set_error("tlm_rmsnorm: dtype %d unsupported (F16, BF16 or F32)", dtype);
    return TLM_EUNSUPPORTED;
  }
  if (rows == 0) return TLM_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TLM_F32) return dispatch_f32(x, w, y, rows, cols, eps, s);
  return dtype == TLM_BF16 ? dispatch<true>(x, w, y, rows, cols, eps, s)
                           : dispatch<false>(x, w, y, rows, cols, eps, s);
}
