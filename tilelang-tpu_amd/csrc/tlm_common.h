// Shared device/host helpers for the gfx950 kernels of libtlmi355x.so.
// Everything here is CDNA4-only: 64-lane wavefronts, MFMA builtins, no portability layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/tlmi355x.h"

// ---------------------------------------------------------------------------------------------
// Vector types (clang ext_vector_type: these are what the MFMA builtins take).
typedef _Float16 f16;
typedef __bf16 bf16;
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));

#define TLM_DEV __device__ __forceinline__

// ---------------------------------------------------------------------------------------------
// Scalar conversions. bf16/fp16 are handled as raw 16-bit patterns so that rounding is explicit.

TLM_DEV float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 with round-to-nearest-even; NaN stays NaN (quiet bit forced).
TLM_DEV uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

TLM_DEV float f16_bits_to_f32(uint32_t b) {
  union { uint16_t u; _Float16 h; } c;
  c.u = (uint16_t)b;
  return (float)c.h;
}

// fp32 -> fp16, round-to-nearest-even (v_cvt_f16_f32 honours the RNE default mode).
TLM_DEV uint32_t f32_to_f16_bits(float f) {
  union { uint16_t u; _Float16 h; } c;
  c.h = (_Float16)f;
  return c.u;
}

// Element type traits for the 16-bit storage types. IS_BF16 selects the format.
template <bool IS_BF16>
struct h16 {
  static TLM_DEV float lo(uint32_t w) {
    return IS_BF16 ? bf16_bits_to_f32(w & 0xffffu) : f16_bits_to_f32(w & 0xffffu);
  }
  static TLM_DEV float hi(uint32_t w) {
    return IS_BF16 ? __uint_as_float(w & 0xffff0000u) : f16_bits_to_f32(w >> 16);
  }
  // Two floats -> two 16-bit values in one dword, round-to-nearest-even
  // (one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 on gfx950).
  static TLM_DEV uint32_t pack(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    if constexpr (IS_BF16) {
      typedef __bf16 o2 __attribute__((ext_vector_type(2)));
      o2 v = __builtin_convertvector((f2){a, b}, o2);
      return __builtin_bit_cast(uint32_t, v);
    } else {
      typedef _Float16 o2 __attribute__((ext_vector_type(2)));
      o2 v = __builtin_convertvector((f2){a, b}, o2);
      return __builtin_bit_cast(uint32_t, v);
    }
  }
  static TLM_DEV float to_f32(uint32_t b16) {
    return IS_BF16 ? bf16_bits_to_f32(b16) : f16_bits_to_f32(b16);
  }
  static TLM_DEV uint32_t from_f32(float f) {
    return IS_BF16 ? f32_to_bf16_bits(f) : f32_to_f16_bits(f);
  }
};

// ---------------------------------------------------------------------------------------------
// Wavefront reductions (64 lanes). xor-shuffles compile to DPP / ds_swizzle / ds_bpermute.
TLM_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
TLM_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// exp(x) through the hardware base-2 exponential: v_exp_f32(x * log2 e).
TLM_DEV float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
TLM_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum of x over lanes l and l ^ 32 through v_permlane32_swap (a VALU op; __shfl_xor would
// be an LDS round trip). Both results are symmetric in the two lane halves.
TLM_DEV float xhalf_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
TLM_DEV float xhalf_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Non-temporal (streaming) 16-byte global accesses for single-use data.
TLM_DEV u32x4 ld_nt(const u32x4* p) { return __builtin_nontemporal_load(p); }
TLM_DEV void st_nt(u32x4* p, u32x4 v) { __builtin_nontemporal_store(v, p); }

// 16-byte accesses with an explicit cache policy CP (gfx950 bits: sc0 = 1, nt = 2, sc1 = 16)
// through a raw buffer descriptor at the wave-uniform address `base`; `off` is the lane's byte
// offset from it (below 2^31). CP_GLOBAL / CP_GLOBAL_NT select a plain / non-temporal global
// access instead.
constexpr int CP_GLOBAL_NT = -1, CP_GLOBAL = -2;
constexpr int CP_PLAIN = 0, CP_NT = 2, CP_SC01 = 17, CP_NT_SC01 = 19;
TLM_DEV __amdgpu_buffer_rsrc_t stream_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, 0x7fffffff, 0x00020000);
}
template <int CP>
TLM_DEV void st_cp(void* base, int off, u32x4 v) {
  if constexpr (CP == CP_GLOBAL_NT)
    __builtin_nontemporal_store(v, (u32x4*)((char*)base + off));
  else if constexpr (CP == CP_GLOBAL)
    *(u32x4*)((char*)base + off) = v;
  else
    __builtin_amdgcn_raw_buffer_store_b128(v, stream_rsrc(base), off, 0, CP);
}
template <int CP>
TLM_DEV u32x4 ld_cp(const void* base, int off) {
  if constexpr (CP == CP_GLOBAL_NT)
    return __builtin_nontemporal_load((const u32x4*)((const char*)base + off));
  else if constexpr (CP == CP_GLOBAL)
    return *(const u32x4*)((const char*)base + off);
  else
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(stream_rsrc(base), off,
                                                                           0, CP));
}

// Stores of a split program's partials (glse / Output_partial) in its dtype, PK: 0 fp16, 1 bf16,
// 2 fp32 (stored unrounded). round() and put4() return the values as a later read gives them back.
template <int PK>
struct part_store {
  static TLM_DEV float round(float x) {
    if constexpr (PK == 2) return x;
    else return h16<PK == 1>::to_f32(h16<PK == 1>::from_f32(x));
  }
  static TLM_DEV void put_lse(void* g, int64_t i, float x) {
    if constexpr (PK == 2) ((float*)g)[i] = x;
    else ((uint16_t*)g)[i] = (uint16_t)h16<PK == 1>::from_f32(x);
  }
  static TLM_DEV f32x4 put4(void* p, int64_t i, f32x4 v) {
    if constexpr (PK == 2) {
      *(f32x4*)((float*)p + i) = v;
      return v;
    } else {
      using H = h16<PK == 1>;
      const u32x2 pk = {H::pack(v[0], v[1]), H::pack(v[2], v[3])};
      *(u32x2*)((uint16_t*)p + i) = pk;
      return f32x4{H::lo(pk[0]), H::hi(pk[0]), H::lo(pk[1]), H::hi(pk[1])};
    }
  }
};

// ---------------------------------------------------------------------------------------------
// Host-side error plumbing (defined in tlm_capi.hip).
void tlm_set_error(const char* fmt, ...);
int tlm_hip_fail(hipError_t e, const char* what);

#define TLM_HIP_CHECK(call)                                     \
  do {                                                          \
    hipError_t _e = (call);                                     \
    if (_e != hipSuccess) return tlm_hip_fail(_e, #call);       \
  } while (0)

// Launch-error check after a <<<>>> launch.
#define TLM_LAUNCH_CHECK(name)                                  \
  do {                                                          \
    hipError_t _e = hipGetLastError();                          \
    if (_e != hipSuccess) return tlm_hip_fail(_e, name);        \
  } while (0)

static inline bool tlm_aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }
