// FP8 GEMM C = A * B^T on gfx950 MFMA: A [M, K] and B [N, K] in OCP e4m3 or e5m2, fp32
// accumulation, C in fp32 / fp16 / bf16 / the input fp8 format.
//
// Reference program: examples/gemm_fp8/example_tilelang_gemm_fp8.py:17-37 (T.gemm with
// transpose_B=True into a float fragment, copied out to an fp8 C; checked against
// (a.half() @ b.half().T).to(fp8), :46-55) and example_tilelang_gemm_fp8_2xAcc.py:10-50 (the same
// product kept in fp32: C is float). The two-level accumulation of the 2xAcc program is a
// Hopper precision workaround; v_mfma_f32_16x16x128_f8f6f4 accumulates every product in fp32.
//
// Design: the 256x256 ping-pong of gemm_256x256 (tlm_gemm.hip) at one byte per element. A k-tile
// is 128 k = 128 bytes per row, the same LDS tile and LDS-DMA pattern as a 64-k 16-bit tile, and
// one v_mfma_f32_16x16x128_f8f6f4 covers the whole k-tile for a 16x16 output tile at twice the
// 16-bit FLOP rate. Each lane holds 32 bytes of its row (A) / column (B) l % 16: the 16-byte
// chunks q and q + 4 of the row, q = l / 16.
#include "tlm_common.h"

#include <type_traits>

namespace {

constexpr int BM = 256, BN = 256, BKB = 128;  // BKB: k per tile = bytes per tile row
constexpr int NTHREADS = 512;
constexpr int RSRC_WORD3 = 0x00020000;
constexpr uint32_t OOB = 0xfffffff0u;
constexpr int ST = BM * BKB;  // bytes per stage (A or B^T)
constexpr int NST_A = 2, NST_B = 3;
constexpr int SMEM = (NST_A + NST_B) * ST;  // 160 KB

// FMT: 0 = e4m3, 1 = e5m2 (the cbsz / blgp format codes of the f8f6f4 MFMA)
template <int FMT>
TLM_DEV f32x4 mma8(i32x8 a, i32x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FMT, FMT, 0, 0, 0, 0);
}

TLM_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
TLM_DEV u32x4 lds_b128(const void* p) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(lds_addr(p)) : "memory");
  return r;
}
template <int N>
TLM_DEV void lgkm_wait() {
  static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
  __builtin_amdgcn_s_waitcnt(0xc07f | (N << 8));
}
TLM_DEV void order_after(u32x4& a) { asm volatile("" : "+v"(a)); }
TLM_DEV void barrier_lds() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
TLM_DEV void wait_dma() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0x3f70);
  __builtin_amdgcn_sched_barrier(0);
}
TLM_DEV i32x8 cat8(u32x4 lo, u32x4 hi) {
  return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
               (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// [rows][128 k] tiles, 16-byte chunk c of row r at c ^ ((r >> 1) & 7): a 16-lane ds_read_b128
// phase covers 16 rows of one chunk column (conflict free), each LDS-DMA instruction 1 KB.
TLM_DEV int swz_rows(int r) { return (r >> 1) & 7; }

TLM_DEV void tile_of(int wg, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int lin = wg;
  if (total % 8 == 0) lin = (wg % 8) * (total / 8) + wg / 8;
  constexpr int GROUP_M = 4;
  const int per_group = GROUP_M * tiles_n;
  const int g = lin / per_group;
  const int first_m = g * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  const int r = lin % per_group;
  tm = first_m + r % gm;
  tn = r / gm;
}

template <int OUT>
TLM_DEV void store_out(void* C, int64_t idx, float v) {
  if constexpr (OUT == TLM_F32) {
    ((float*)C)[idx] = v;
  } else if constexpr (OUT == TLM_BF16) {
    ((uint16_t*)C)[idx] = (uint16_t)f32_to_bf16_bits(v);
  } else if constexpr (OUT == TLM_F16) {
    ((uint16_t*)C)[idx] = (uint16_t)f32_to_f16_bits(v);
  } else if constexpr (OUT == TLM_F8E4M3) {  // round to nearest even, no saturation (torch's cast)
    ((uint8_t*)C)[idx] = (uint8_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, 0.f, 0, false);
  } else {
    ((uint8_t*)C)[idx] = (uint8_t)__builtin_amdgcn_cvt_pk_bf8_f32(v, 0.f, 0, false);
  }
}

template <int FMT, int OUT>
__global__ __launch_bounds__(NTHREADS, 1) void gemm8_256x256(const uint8_t* __restrict__ A,
                                                            const uint8_t* __restrict__ B,
                                                            void* __restrict__ C, int M, int N,
                                                            int K) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2;  // 128-row half
  const int wn = wave & 3;   // 64-column quarter
  int tm, tn;
  tile_of(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int KT = (K + BKB - 1) / BKB;

  struct Dma {
    const uint8_t* base[2];
    uint8_t* st[2];
  };
  auto sa_of = [&](int kt) { return smem + (kt % NST_A) * ST; };
  auto sb_of = [&](int kt) { return smem + NST_A * ST + (kt % NST_B) * ST; };
  auto dma_setup = [&](int kt) {
    const int k0 = kt * BKB;
    return Dma{{A + ((int64_t)m0 * K + k0), B + ((int64_t)n0 * K + k0)},
               {sa_of(kt), sb_of(kt)}};
  };
  // instruction ins (0..31) of operand op (0 = A, 1 = B): 8 rows of 128 bytes; chunks beyond K
  // or rows beyond M / N read zeros through the out-of-range offset
  auto dma = [&](const Dma& dd, auto OPc, int ins, int kmax) {
    constexpr int op = decltype(OPc)::value;
    const int r = 8 * ins + (lane >> 3);
    const int c = (lane & 7) ^ swz_rows(r);
    const bool ok = (op == 0 ? m0 + r < M : n0 + r < N) && 16 * c < kmax;
    const uint32_t off = (uint32_t)(r * K + 16 * c);
    uint8_t* dst = dd.st[op] + ins * 1024;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)dd.base[op], (short)0, 0x7ffffff0, RSRC_WORD3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)dst, 16,
                                             ok ? off : OOB, 0, 0, 0);
  };
  // a group's share of one operand stage: wave wl of the group issues instructions
  // 8 wl .. 8 wl + 7
  using OpA = std::integral_constant<int, 0>;
  using OpB = std::integral_constant<int, 1>;
  auto issue_op = [&](int kt, auto OPc) {
    const Dma dd = dma_setup(kt);
    const int kmax = min(BKB, K - kt * BKB);
#pragma unroll
    for (int j = 0; j < 8; ++j) dma(dd, OPc, 8 * (wave & 3) + j, kmax);
  };

  f32x4 acc[8][4];  // [16-row tile mt][16-column tile nt] of the wave's 128 x 64 sub-tile
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{};

  // v_mfma_f32_16x16x128_f8f6f4: lane l holds row (A) / column (B) l % 16 and 32 of the 128 k;
  // any assignment of k to lanes gives the same product when A and B use the same one. Lane
  // group q = l / 16 takes the 16-byte chunks q and q + 4 of the 128-byte row, so a 16-lane
  // read covers 16 rows of one chunk column (conflict free under the row swizzle). The 16x16
  // shape draws less power per FLOP than 32x32 (a higher sustained clock).
  const int q4 = lane >> 4;
  const int sw = (lane >> 1) & 7;
  const int a_row = (wm * 128 + (lane & 15)) * BKB;  // + mt * 16 rows
  const int b_row = (wn * 64 + (lane & 15)) * BKB;   // + nt * 16 rows

  // Ping-pong of the two waves on each SIMD (groups of 4), as in gemm_256x256: one reads the
  // next k-tile's A operands and its first B operand while the other issues MFMAs; every phase
  // ends with a workgroup barrier. LDS-DMA is issued only in load phases: group 0 fills A of
  // k-tile kt + 1 in phase 2 kt (its stage held A of kt - 1, last read in phase 2 kt - 1),
  // group 1 fills B of kt + 2 in phase 2 kt + 1 (its stage held B of kt - 1, last read in
  // phase 2 kt), so each phase carries one 32 KB operand stage of DMA.
  const int grp = wave >> 2;
  u32x4 aop[8][2];  // [mt][chunk] of the k-tile
  u32x4 bop0[2];    // first B operand of the k-tile (read in the load phase)
  auto chunk = [&](int p) { return 16 * ((4 * p + q4) ^ sw); };
  auto readb = [&](int kt, int nt, u32x4 (&o)[2]) {
    const uint8_t* sb = sb_of(kt);
#pragma unroll
    for (int p = 0; p < 2; ++p) o[p] = lds_b128(sb + b_row + nt * 16 * BKB + chunk(p));
  };
  // the wave's 8 instructions of the phase, two after every four operand reads
  auto dma_pair = [&](const Dma& dd, int dma_kt, auto OPc, int q) {
    if (dma_kt >= 0) {
      const int kmax = min(BKB, K - dma_kt * BKB);
      dma(dd, OPc, 8 * (wave & 3) + 2 * q, kmax);
      dma(dd, OPc, 8 * (wave & 3) + 2 * q + 1, kmax);
    }
  };
  auto load_phase = [&](int kt, int dma_kt, auto OPc) {
    const uint8_t* sa = sa_of(kt);
    const Dma dd = dma_setup(dma_kt < 0 ? 0 : dma_kt);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int m2 = 0; m2 < 2; ++m2)
#pragma unroll
        for (int p = 0; p < 2; ++p)
          aop[2 * q + m2][p] = lds_b128(sa + a_row + (2 * q + m2) * 16 * BKB + chunk(p));
      dma_pair(dd, dma_kt, OPc, q);
    }
    readb(kt, 0, bop0);
    lgkm_wait<0>();
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int p = 0; p < 2; ++p) order_after(aop[mt][p]);
    order_after(bop0[0]);
    order_after(bop0[1]);
  };
  auto compute_phase = [&](int kt) {
    u32x4 b[3][2];  // ring: operand nt in b[nt % 3], read two ahead
    b[0][0] = bop0[0];
    b[0][1] = bop0[1];
    readb(kt, 1, b[1]);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      if (nt + 2 < 4) readb(kt, nt + 2, b[(nt + 2) % 3]);
      // operand nt has landed; the reads of nt + 1 and nt + 2 (2 instructions each) stay in flight
      if (nt + 2 < 4)
        lgkm_wait<4>();
      else if (nt + 1 < 4)
        lgkm_wait<2>();
      else
        lgkm_wait<0>();
      order_after(b[nt % 3][0]);
      order_after(b[nt % 3][1]);
#pragma unroll
      for (int mt = 0; mt < 8; ++mt)
        acc[mt][nt] = mma8<FMT>(cat8(aop[mt][0], aop[mt][1]), cat8(b[nt % 3][0], b[nt % 3][1]),
                                acc[mt][nt]);
    }
  };
  // prologue: A of k-tile 0 (group 0), B of k-tiles 0 and 1 (group 1)
  if (grp == 0) {
    issue_op(0, OpA{});
  } else {
    issue_op(0, OpB{});
    if (1 < KT) issue_op(1, OpB{});
  }
  wait_dma();
  barrier_lds();
  if (grp == 0) {
    for (int kt = 0; kt < KT; ++kt) {
      load_phase(kt, kt + 1 < KT ? kt + 1 : -1, OpA{});  // phase 2 kt (+ A of kt + 1)
      barrier_lds();
      compute_phase(kt);  // phase 2 kt + 1
      wait_dma();         // A of kt + 1 landed
      barrier_lds();
    }
    barrier_lds();  // phase 2 KT: group 1 computes the last k-tile
  } else {
    barrier_lds();  // phase 0
    for (int kt = 0; kt < KT; ++kt) {
      const bool dma = kt + 2 < KT;
      load_phase(kt, dma ? kt + 2 : -1, OpB{});  // phase 2 kt + 1 (+ B of kt + 2)
      // B of kt + 1 (issued one load phase earlier, or in the prologue) has landed
      __builtin_amdgcn_sched_barrier(0);
      if (dma)
        __builtin_amdgcn_s_waitcnt(0x3f78);  // vmcnt(8): this phase's 8 may stay in flight
      else
        __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)
      __builtin_amdgcn_sched_barrier(0);
      barrier_lds();
      compute_phase(kt);  // phase 2 kt + 2
      barrier_lds();
    }
  }

  // epilogue: lane holds column (lane & 15) of each 16x16 tile, rows 4 (lane / 16) + i.
  // fp32 C with N % 4 == 0 and C 16-byte aligned: the wave's 128 x 64 sub-tile goes through its
  // own 16 KB of LDS in two 64-row halves (the stages are free: the last barrier ended every
  // operand read and no LDS-DMA is in flight) and leaves as 16-byte row vectors, one 256-byte
  // row per 16 lanes, instead of 4-byte stores. Stage row r holds 64 floats (16 chunks of 16
  // bytes); chunk c sits at c ^ 4((r / 4) % 4), so the four row groups of one 4-byte write land
  // in four different 64-byte bank windows and a 16-lane read covers one row. The row stores
  // are non-temporal (C is not read again; ~1.5% faster per launch at 4096^3).
  if constexpr (OUT == TLM_F32) {
    if (N % 4 == 0 && ((uintptr_t)C & 15) == 0) {
      float* stg = (float*)smem + wave * (64 * 64);
      float* Cf = (float*)C;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int nt = 0; nt < 4; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int r = m * 16 + 4 * (lane >> 4) + i, c = nt * 16 + (lane & 15);
              stg[r * 64 + 4 * ((c >> 2) ^ (4 * ((r >> 2) & 3))) + (c & 3)] =
                  acc[4 * h + m][nt][i];
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int it = 0; it < 16; ++it) {
          const int idx = it * 64 + lane, r = idx >> 4, c4 = idx & 15;
          const u32x4 v = *(const u32x4*)(stg + r * 64 + 4 * (c4 ^ (4 * ((r >> 2) & 3))));
          const int row = m0 + wm * 128 + 64 * h + r, col = n0 + wn * 64 + 4 * c4;
          if (row < M && col < N) st_nt((u32x4*)(Cf + (int64_t)row * N + col), v);
        }
        // the second half overwrites the stage only after every lane has read the first
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
      return;
    }
  }
#pragma unroll
  for (int mt = 0; mt < 8; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int col = n0 + wn * 64 + nt * 16 + (lane & 15);
      if (col >= N) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = m0 + wm * 128 + mt * 16 + 4 * (lane >> 4) + i;
        if (row < M) store_out<OUT>(C, (int64_t)row * N + col, acc[mt][nt][i]);
      }
    }
}

// fp8 byte -> float, exact (e4m3: bias 7, no infinities, 0x7f / 0xff NaN; e5m2: IEEE-like)
template <int FMT>
TLM_DEV float f8_to_f32(uint8_t b) {
  const uint32_t s = (b & 0x80u) << 24;
  if constexpr (FMT == 0) {
    const uint32_t e = (b >> 3) & 15, m = b & 7;
    if (e == 15 && m == 7) return __uint_as_float(0x7fc00000u | s);
    if (e == 0) return __uint_as_float(s) + (s ? -1.f : 1.f) * (float)m * 0x1p-9f;
    return __uint_as_float(s | ((e + 120) << 23) | (m << 20));
  } else {
    const uint32_t e = (b >> 2) & 31, m = b & 3;
    if (e == 31) return __uint_as_float(s | 0x7f800000u | (m ? 0x400000u : 0u));
    if (e == 0) return __uint_as_float(s) + (s ? -1.f : 1.f) * (float)m * 0x1p-16f;
    return __uint_as_float(s | ((e + 112) << 23) | (m << 21));
  }
}

// Any shape and either B layout: one thread per output, fp32 accumulation in k order.
template <int FMT, bool TRANS_B, int OUT>
__global__ __launch_bounds__(256) void gemm8_generic(const uint8_t* __restrict__ A,
                                                     const uint8_t* __restrict__ B,
                                                     void* __restrict__ C, int M, int N, int K) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int m = (int)(idx / N), n = (int)(idx % N);
  float s = 0.f;
  for (int k = 0; k < K; ++k) {
    const float a = f8_to_f32<FMT>(A[(int64_t)m * K + k]);
    const float b = f8_to_f32<FMT>(TRANS_B ? B[(int64_t)n * K + k] : B[(int64_t)k * N + n]);
    s = fmaf(a, b, s);
  }
  store_out<OUT>(C, idx, s);
}

template <int FMT, int OUT>
int launch(const void* A, const void* B, void* C, int M, int N, int K, bool trans_b,
           hipStream_t s) {
  // 32-bit LDS-DMA byte offsets r * K + 16 c within a 256-row panel stay below the
  // descriptor's num_records (2^31 - 16): K < 2^23
  const bool tiled = trans_b && M > 16 && K % 16 == 0 && K < (1 << 23) && tlm_aligned(A, 16) &&
                     tlm_aligned(B, 16);
  if (tiled) {
    const int64_t tiles = (int64_t)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    gemm8_256x256<FMT, OUT><<<(unsigned)tiles, NTHREADS, 0, s>>>(
        (const uint8_t*)A, (const uint8_t*)B, C, M, N, K);
  } else {
    const int64_t n = (int64_t)M * N;
    if (trans_b)
      gemm8_generic<FMT, true, OUT><<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
          (const uint8_t*)A, (const uint8_t*)B, C, M, N, K);
    else
      gemm8_generic<FMT, false, OUT><<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
          (const uint8_t*)A, (const uint8_t*)B, C, M, N, K);
  }
  TLM_LAUNCH_CHECK("tlm_gemm_fp8");
  return TLM_OK;
}

template <int FMT>
int by_out(const void* A, const void* B, void* C, int M, int N, int K, bool tb, int out,
           hipStream_t s) {
  switch (out) {
    case TLM_F32: return launch<FMT, TLM_F32>(A, B, C, M, N, K, tb, s);
    case TLM_F16: return launch<FMT, TLM_F16>(A, B, C, M, N, K, tb, s);
    case TLM_BF16: return launch<FMT, TLM_BF16>(A, B, C, M, N, K, tb, s);
    case TLM_F8E4M3: return launch<FMT, TLM_F8E4M3>(A, B, C, M, N, K, tb, s);
    default: return launch<FMT, TLM_F8E5M2>(A, B, C, M, N, K, tb, s);
  }
}

}  // namespace

extern "C" int tlm_gemm_fp8(const void* A, const void* B, void* C, int64_t M, int64_t N,
                            int64_t K, int in_dtype, int out_dtype, int trans_b, void* stream) {
  if (!A || !B || !C) {
    tlm_set_error("tlm_gemm_fp8: null pointer argument");
    return TLM_EINVAL;
  }
  if (M < 0 || N < 0 || K < 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX ||
      M * N > ((int64_t)1 << 40) || (M > 0 && K > 0 && (M - 1) * K + K > INT32_MAX) ||
      (N > 0 && K > 0 && (N - 1) * K + K > INT32_MAX)) {
    tlm_set_error("tlm_gemm_fp8: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                  (long long)K);
    return TLM_EINVAL;
  }
  if (trans_b != 0 && trans_b != 1) {
    tlm_set_error("tlm_gemm_fp8: trans_b must be 0 or 1");
    return TLM_EINVAL;
  }
  if (in_dtype != TLM_F8E4M3 && in_dtype != TLM_F8E5M2) {
    tlm_set_error("tlm_gemm_fp8: in_dtype %d unsupported (F8E4M3 or F8E5M2)", in_dtype);
    return TLM_EUNSUPPORTED;
  }
  if (out_dtype != TLM_F32 && out_dtype != TLM_F16 && out_dtype != TLM_BF16 &&
      out_dtype != in_dtype) {
    tlm_set_error("tlm_gemm_fp8: out_dtype %d unsupported (F32, F16, BF16 or the input format)",
                  out_dtype);
    return TLM_EUNSUPPORTED;
  }
  const int osz =
      out_dtype == TLM_F32 ? 4 : (out_dtype == TLM_F16 || out_dtype == TLM_BF16) ? 2 : 1;
  if (!tlm_aligned(C, osz)) {
    tlm_set_error("tlm_gemm_fp8: misaligned C");
    return TLM_EINVAL;
  }
  if (M == 0 || N == 0) return TLM_OK;
  hipStream_t s = (hipStream_t)stream;
  const int m = (int)M, n = (int)N, k = (int)K;
  return in_dtype == TLM_F8E4M3 ? by_out<0>(A, B, C, m, n, k, trans_b != 0, out_dtype, s)
                                : by_out<1>(A, B, C, m, n, k, trans_b != 0, out_dtype, s);
}
