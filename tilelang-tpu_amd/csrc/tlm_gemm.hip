// GEMM C = A * B on gfx950 MFMA (fp16 / bf16 in, fp32 accumulate, one rounding on store).
//
// Reference semantics: ppl_gemm with transpose_B=False is C += A*B into an fp32 tile
// (src/target/codegen_ppl.cc:1244-1279, tpu_bdc_fp_mm), the matmul demo fills C with 0, loops over
// K and casts the fp32 tile to the output dtype once (tpu_demo/matmul/tpu_test_matmul_fp16.py:19-29).
//
// Main kernel (any M, N; K % 8 == 0, N % 8 == 0 for row-major B):
//   * 256x256 output tile per workgroup, BK = 64, 512 threads = 8 waves of 128x64 sub-tiles;
//   * v_mfma_f32_16x16x32_{f16,bf16}: per wave 8x4 accumulator tiles = 128 fp32 VGPRs;
//   * A tiles [256][64] and B tiles [64][256] (row-major B kept row-major; [256][64] for B^T)
//     are filled by buffer_load ... lds (16 bytes per lane straight into LDS, no VGPR staging)
//     into unpadded, XOR-swizzled stages (2 for A, 3 for B: 160 KB); lanes whose chunk lies
//     outside the matrix read zeros through the buffer descriptor's bounds;
//   * the two waves on each SIMD (groups of 4) run half a k-tile apart: one reads the next
//     k-tile's operands from LDS while the other issues MFMAs; LDS-DMA is issued only by the
//     reading group, between its operand reads (group 0 fills A stages, group 1 B stages);
//   * the B operand (8 consecutive k of one column per lane) is read with ds_read_b64_tr_b16,
//     which transposes 4x16 blocks of 16-bit values across each 16-lane group, so B needs no
//     transpose in registers or in a separate pass;
//   * workgroup -> tile order is XCD-aware: consecutive workgroup ids land on different XCDs
//     (round-robin dispatch), so ids are regrouped to give each XCD a compact block of tiles
//     that shares A row-panels and B column-panels in that XCD's L2.
// Skinny kernels (M <= 16): gemm_skinny_split for row-major B, gemm_skinny for B^T and the shapes
// or streams the split kernel does not take; see below.
#include "tlm_common.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int NTHREADS = 512;

template <bool BF16>
struct mfma16_t;
template <>
struct mfma16_t<false> {
  typedef f16x8 v8;
  static TLM_DEV f32x4 mma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct mfma16_t<true> {
  typedef bf16x8 v8;
  static TLM_DEV f32x4 mma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// Transposed LDS read: 4 k-rows starting at `p` (lane's own row/column chunk, see call site).
TLM_DEV s16x4 lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

template <typename V8>
TLM_DEV V8 cat4(s16x4 lo, s16x4 hi) {
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(V8, v);
}

// Tile order: regroup workgroup ids so each XCD (id % 8) gets a contiguous range of the
// grouped (GROUP_M rows of tiles at a time) tile sequence.
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
  if constexpr (OUT == TLM_F32)
    ((float*)C)[idx] = v;
  else if constexpr (OUT == TLM_BF16)
    ((uint16_t*)C)[idx] = (uint16_t)f32_to_bf16_bits(v);
  else
    ((uint16_t*)C)[idx] = (uint16_t)f32_to_f16_bits(v);
}

// LDS access as inline asm: compiler-generated LDS reads may be made to wait for every
// outstanding LDS-DMA load (including the prefetch of the next k-tile) when the compiler cannot
// prove that they touch the other stage. Waits are explicit (lgkm_wait + order_after).
TLM_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
TLM_DEV u32x4 lds_b128(const void* p) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(lds_addr(p)) : "memory");
  return r;
}
TLM_DEV u32x2 lds_tr16(const void* p) {
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(lds_addr(p)) : "memory");
  return r;
}
TLM_DEV void lgkm_wait(int n) {  // lgkmcnt(n); n a compile-time constant after unrolling
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0xc07f); break;
    case 1: __builtin_amdgcn_s_waitcnt(0xc17f); break;
    case 2: __builtin_amdgcn_s_waitcnt(0xc27f); break;
    case 4: __builtin_amdgcn_s_waitcnt(0xc47f); break;
    case 8: __builtin_amdgcn_s_waitcnt(0xc87f); break;
    default: __builtin_amdgcn_s_waitcnt(0xc07f); break;
  }
}
TLM_DEV void order_after(u32x4& a) { asm volatile("" : "+v"(a)); }
// Phase boundaries: sched_barrier keeps the scheduler from moving instructions (MFMAs only touch
// registers) across the wait or the barrier.
TLM_DEV void barrier_lds() {  // workgroup barrier; LDS-DMA loads stay in flight
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
TLM_DEV void wait_dma() {  // this thread's LDS-DMA loads have landed
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0x3f70);
  __builtin_amdgcn_sched_barrier(0);
}

constexpr int RSRC_WORD3 = 0x00020000;  // raw buffer, 32-bit data format
constexpr uint32_t OOB = 0xfffffff0u;   // offset past num_records: the load returns zeros
// LDS tiles (16-bit elements, no padding), 16-byte chunks XOR-swizzled so that the MFMA operand
// reads are bank-conflict free and every LDS-DMA instruction fills 1 KB of contiguous LDS:
//   * [rows][64 k] tiles (A, and B^T): chunk c of row r at c ^ ((r >> 1) & 7);
//     a 16-lane ds_read_b128 phase covers rows r0..r0+15 of one chunk column;
//   * [64 k][256 n] row-major B: chunk c of row k at c ^ (2 (k & 3) + 8 ((k >> 3) & 1)); a
//     32-lane ds_read_b64_tr_b16 phase covers k-rows k0..k0+3 and k0+8..k0+11 of the same 32
//     bytes of columns (two 16x16x32 operand groups): 16 distinct chunk positions.
TLM_DEV int swz_rows(int r) { return (r >> 1) & 7; }
TLM_DEV int swz_k(int k) { return 2 * (k & 3) + 8 * ((k >> 3) & 1); }
constexpr int ST_A = BM * BK * 2;  // bytes per stage of A
constexpr int ST_B = BK * BN * 2;  // bytes per stage of B (either layout)
constexpr int NST_A = 2, NST_B = 3;
constexpr int SMEM = NST_A * ST_A + NST_B * ST_B;  // 160 KB

template <bool BF16, bool TRANS_B, int OUT>
__global__ __launch_bounds__(NTHREADS, 1) void gemm_256x256(const uint16_t* __restrict__ A,
                                                           const uint16_t* __restrict__ B,
                                                           void* __restrict__ C, int M, int N,
                                                           int K) {
  using MT = mfma16_t<BF16>;
  using v8 = typename MT::v8;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2;  // 0..1: 128-row half
  const int wn = wave & 3;   // 0..3: 64-col quarter
  int tm, tn;
  tile_of(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int KT = (K + BK - 1) / BK;

  // ---- LDS-DMA fill: a 32 KB stage is 32 wave-instructions of 1 KB; instruction `ins` covers
  // LDS slots [64 ins, 64 ins + 64) of its operand. Lanes whose chunk lies outside A, B (rows
  // against M / N, columns against K) read zeros.
  struct Dma {  // the k-tile's A and B base addresses and LDS destinations
    const uint16_t* base[2];
    uint8_t* st[2];
  };
  auto sa_of = [&](int kt) { return smem + (kt % NST_A) * ST_A; };
  auto sb_of = [&](int kt) { return smem + NST_A * ST_A + (kt % NST_B) * ST_B; };
  auto dma_setup = [&](int kt) {
    const int k0 = kt * BK;
    return Dma{{A + ((int64_t)m0 * K + k0),
                TRANS_B ? B + ((int64_t)n0 * K + k0) : B + ((int64_t)k0 * N + n0)},
               {sa_of(kt), sb_of(kt)}};
  };
  // kmax: number of valid k (columns for A / B^T, rows for row-major B) in this k-tile;
  // op: 0 = A, 1 = B
  auto dma = [&](const Dma& dd, auto OPc, int ins, int kmax) {
    constexpr int op = decltype(OPc)::value;
    uint32_t off;
    bool ok;
    if constexpr (op == 0 || TRANS_B) {  // [rows][64 k]: 8 rows of 128 bytes
      const int r = 8 * ins + (lane >> 3);
      const int c = (lane & 7) ^ swz_rows(r);
      ok = (op == 0 ? m0 + r < M : n0 + r < N) && 8 * c < kmax;
      off = (uint32_t)(r * K + 8 * c) * 2u;
    } else {  // row-major B [64 k][256 n]: 2 k-rows of 512 bytes
      const int k = 2 * ins + (lane >> 5);
      const int c = (lane & 31) ^ swz_k(k);
      ok = n0 + 8 * c < N && k < kmax;
      off = (uint32_t)(k * N + 8 * c) * 2u;
    }
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
    const int kmax = min(BK, K - kt * BK);
#pragma unroll
    for (int j = 0; j < 8; ++j) dma(dd, OPc, 8 * (wave & 3) + j, kmax);
  };

  f32x4 acc[8][4];  // [16-row tile mt][16-column tile nt] of the wave's 128 x 64 sub-tile
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{};

  // ---- per-lane operand read offsets (bytes within a stage). v_mfma_f32_16x16x32: lane l holds
  // row (A) / column (B) l % 16 and k = 8 (l / 16) .. + 7 of the 32-k step. The 16x16 shape
  // keeps the same LDS traffic per FLOP as 32x32x16 and draws less power per FLOP: a pure MFMA
  // loop on all CUs settled at 2.39 GHz against 2.22 GHz for 32x32x16 at the same efficiency
  // per cycle.
  const int q4 = lane >> 4;                                    // k chunk within the step
  const int sw = (lane >> 1) & 7;                              // swz_rows of this lane's rows
  const int a_row = (wm * 128 + (lane & 15)) * (BK * 2);       // + mt * 16 rows
  const int bt_row = (wn * 64 + (lane & 15)) * (BK * 2);       // + nt * 16 rows (B^T)
  // row-major B through ds_read_b64_tr_b16: 16-lane group h reads k-rows 8 h + j / 4 (+ 4 for
  // the second read, + 32 for the second k-step); lane j addresses the 8 bytes at columns
  // 16 nt + 4 (j % 4) and receives column j of the four rows
  const int h = lane >> 4, j = lane & 15;
  const int tr_k = 8 * h + (j >> 2);
  const int tr_c = 8 * wn + ((j & 3) >> 1);                    // chunk, + 2 nt
  const int tr_off = tr_k * (BN * 2) + 8 * (j & 1);
  const int tr_sw = swz_k(tr_k);                               // the same for every k-step

  // Ping-pong schedule. The two waves on a SIMD (w and w + 4, groups grp = w / 4) run half a
  // k-tile apart: in each phase one of them issues MFMAs while the other reads the next k-tile's
  // A operands (both k-steps) and first B operand from LDS into registers; the computing wave
  // reads B two operands ahead. Group 0 loads k-tile kt in phase 2 kt and computes it in
  // phase 2 kt + 1; group 1 is one phase later. Every phase ends with a workgroup barrier.
  // A k-tile's A stage is read in phases 2 kt, 2 kt + 1 and its B stage through phase 2 kt + 2,
  // hence 2 A stages and 3 B stages. LDS-DMA is issued only in load phases, where the waves
  // have no MFMAs to delay (issue stalls on the vector memory path, ~80 cycles per 1 KB
  // instruction, measured ~700 cycles per phase when issued from a compute phase): group 0
  // loads A of k-tile kt + 1 in phase 2 kt (its stage held A of kt - 1, read by phase 2 kt - 1),
  // group 1 loads B of k-tile kt + 2 in phase 2 kt + 1 (its stage held B of kt - 1, read by
  // phase 2 kt). A lands within two phases, B within three.
  const int grp = wave >> 2;
  u32x4 aop[BK / 32][8];  // A operands of a whole k-tile: [k-step][mt]
  u32x4 bop0;             // first B operand of the k-tile (read in the load phase)
  // B operand t = 4 ks + nt of k-tile kt
  auto readb = [&](int kt, int t) {
    const uint8_t* sb = sb_of(kt);
    const int ks = t >> 2, nt = t & 3;
    if constexpr (TRANS_B) {
      return lds_b128(sb + bt_row + nt * 16 * BK * 2 + 16 * ((4 * ks + q4) ^ sw));
    } else {
      const uint8_t* q = sb + (32 * ks) * (BN * 2) + tr_off + 16 * ((tr_c + 2 * nt) ^ tr_sw);
      const u32x2 lo = lds_tr16(q);
      const u32x2 hi = lds_tr16(q + 4 * (BN * 2));
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  };
  constexpr int BREADS = TRANS_B ? 1 : 2;  // LDS instructions of readb()
  // The group's 8 LDS-DMA instructions of the phase go two after every four operand reads
  // instead of in one burst. dma_kt < 0: nothing to issue; op: operand of the group.
  auto dma_pair = [&](const Dma& dd, int dma_kt, auto OPc, int q) {
    if (dma_kt >= 0) {
      const int kmax = min(BK, K - dma_kt * BK);
      dma(dd, OPc, 8 * (wave & 3) + 2 * q, kmax);
      dma(dd, OPc, 8 * (wave & 3) + 2 * q + 1, kmax);
    }
  };
  auto load_phase = [&](int kt, int dma_kt, auto OPc) {
    const uint8_t* sa = sa_of(kt);
    const Dma dd = dma_setup(dma_kt < 0 ? 0 : dma_kt);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int m4 = 0; m4 < 4; ++m4) {
          const int mt = 4 * half + m4;
          aop[ks][mt] = lds_b128(sa + a_row + mt * 16 * BK * 2 + 16 * ((4 * ks + q4) ^ sw));
        }
        dma_pair(dd, dma_kt, OPc, 2 * ks + half);
      }
    bop0 = readb(kt, 0);
    lgkm_wait(0);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks)
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) order_after(aop[ks][mt]);
    order_after(bop0);
  };
  auto compute_phase = [&](int kt) {
    constexpr int NB = 4 * (BK / 32);  // B operands per k-tile
    u32x4 b[3];                        // ring: operand t in b[t % 3], read two ahead
    b[0] = bop0;
    b[1] = readb(kt, 1);
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      if (t + 2 < NB) b[(t + 2) % 3] = readb(kt, t + 2);
      // operand t has landed; the reads of t + 1 and t + 2 stay in flight
      const int ahead = (t + 1 < NB ? 1 : 0) + (t + 2 < NB ? 1 : 0);
      lgkm_wait(ahead * BREADS);
      order_after(b[t % 3]);
      const int ks = t >> 2, nt = t & 3;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt)
        acc[mt][nt] = MT::mma(__builtin_bit_cast(v8, aop[ks][mt]),
                              __builtin_bit_cast(v8, b[t % 3]), acc[mt][nt]);
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
  // 16-bit C with N % 8 == 0 and C 16-byte aligned: the wave's 128 x 64 sub-tile is rounded
  // into its own 16 KB of LDS (the operand stages are free: the last barrier ended every operand
  // read and no LDS-DMA is in flight) and written back as 16-byte row vectors, full 128-byte
  // lines per 8 lanes, instead of 2-byte stores. Stage row r holds 64 columns (128 bytes); its 16-byte chunk c sits
  // at c ^ ((r / 4) % 8), so the four row groups of one 2-byte write and the two rows of one
  // 16-lane read hit distinct banks. The row stores are non-temporal (C is not read again;
  // ~1% faster per launch at 4096^3).
  if constexpr (OUT != TLM_F32) {
    if (N % 8 == 0 && ((uintptr_t)C & 15) == 0) {
      uint16_t* stg = (uint16_t*)smem + wave * (128 * 64);
#pragma unroll
      for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = mt * 16 + 4 * (lane >> 4) + i, c = nt * 16 + (lane & 15);
            const float v = acc[mt][nt][i];
            stg[r * 64 + 8 * ((c >> 3) ^ ((r >> 2) & 7)) + (c & 7)] =
                (uint16_t)(OUT == TLM_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
          }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      uint16_t* Cb = (uint16_t*)C;
#pragma unroll
      for (int it = 0; it < 16; ++it) {
        const int idx = it * 64 + lane, r = idx >> 3, c8 = idx & 7;
        const u32x4 v = *(const u32x4*)(stg + r * 64 + 8 * (c8 ^ ((r >> 2) & 7)));
        const int row = m0 + wm * 128 + r, col = n0 + wn * 64 + 8 * c8;
        if (row < M && col < N) st_nt((u32x4*)(Cb + (int64_t)row * N + col), v);
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

// ------------------------------------------------------------------------------------------------
// Skinny GEMM (M <= 16) for B^T and the row-major cases gemm_skinny_split does not take: the
// whole of A fits one MFMA row block, so the kernel streams B.
// Workgroup = 8 waves on a 64-column strip of C; the waves split K into interleaved 32-row
// blocks, each block is one v_mfma_f32_16x16x32 per 16 columns. A operand (row m = lane%16,
// k = 8*(lane/16)..+7) is a direct 16-byte global load. Row-major B goes through a wave-private
// LDS buffer [32][64] and comes back through ds_read_b64_tr_b16; B^T ([N,K]) is loaded straight
// into operand layout. The next block's loads are issued before the current block's MFMAs.
// The 8 partial 16x64 tiles are summed through LDS at the end. B is read once per call, with
// non-temporal loads: 3% faster back to back, and a single launch after a cache flush 27 against
// 48 us at 16 x 14336 x 4096. With nsplit > 1 (B^T with few strips) the workgroups of a strip
// take 1/nsplit of K each and their tiles meet as in gemm_skinny_split (split order, last
// arriver).
constexpr int SS_WAVES = 8;
constexpr int SS_NT = 128;
constexpr int SS_BK = 16;
constexpr int SS_AMAX_K = 2048;  // k range of one workgroup: its A is 64 KB of LDS
constexpr int SS_MAX_SPLIT = 16;
constexpr int SS_SLOTS = 4;
constexpr int SS_MAX_WG = 512;   // workgroups of one call that publish a partial tile
constexpr int SS_PART = 16 * SS_NT;
constexpr int SK_WAVES = 8;
constexpr int SK_NT = 64;
constexpr int SK_BK = 32;
constexpr int SK_BPITCH = SK_NT + 16;  // halves per LDS row of a B block (160 bytes)


template <bool BF16, bool TRANS_B, int OUT>
__global__ __launch_bounds__(64 * SK_WAVES) void gemm_skinny(const uint16_t* __restrict__ A,
                                                            const uint16_t* __restrict__ B,
                                                            void* __restrict__ C, int M, int N,
                                                            int K, int nsplit, float* part,
                                                            unsigned* arrivals) {
  using MT = mfma16_t<BF16>;
  using v8 = typename MT::v8;
  __shared__ __attribute__((aligned(16))) uint16_t sbuf[SK_WAVES][SK_BK * SK_BPITCH];
  __shared__ float red[SK_WAVES][16][SK_NT + 1];
  __shared__ unsigned last_arrival;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nstrips = (N + SK_NT - 1) / SK_NT;
  const int strip = blockIdx.x % nstrips, split = blockIdx.x / nstrips;
  const int n0 = strip * SK_NT;
  const int KBall = (K + SK_BK - 1) / SK_BK;
  const int kb_lo = (int)((int64_t)split * KBall / nsplit);
  const int KB = (int)((int64_t)(split + 1) * KBall / nsplit);  // this split's blocks end
  const int am = lane & 15, ak = 8 * (lane >> 4);
  // row-major B block loads: 32 rows x 64 cols = 4 vectors per lane (rows lane/8 + 8p)
  const int br = lane >> 3, bc = (lane & 7) * 8;
  const int h = lane >> 4, j = lane & 15;

  f32x4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x4{};

  u32x4 ra, rb[4];
  auto load = [&](int kb) {
    const int k0 = kb * SK_BK;
    ra = (am < M && k0 + ak < K) ? *(const u32x4*)(A + (int64_t)am * K + k0 + ak)
                                 : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if constexpr (TRANS_B) {
        const int gn = n0 + 16 * p + am;
        rb[p] = (gn < N && k0 + ak < K) ? ld_nt((const u32x4*)(B + (int64_t)gn * K + k0 + ak))
                                        : u32x4{0, 0, 0, 0};
      } else {
        const int gk = k0 + br + 8 * p, gn = n0 + bc;
        rb[p] = (gk < K && gn < N) ? ld_nt((const u32x4*)(B + (int64_t)gk * N + gn))
                                   : u32x4{0, 0, 0, 0};
      }
    }
  };

  uint16_t* my = sbuf[wave];
  int kb = kb_lo + wave;
  if (kb < KB) load(kb);
  for (; kb < KB; kb += SK_WAVES) {
    const u32x4 ca = ra;
    u32x4 cb[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) cb[p] = rb[p];
    if (kb + SK_WAVES < KB) load(kb + SK_WAVES);
    const v8 av = __builtin_bit_cast(v8, ca);
    if constexpr (TRANS_B) {
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = MT::mma(av, __builtin_bit_cast(v8, cb[t]), acc[t]);
    } else {
#pragma unroll
      for (int p = 0; p < 4; ++p) *(u32x4*)(my + (br + 8 * p) * SK_BPITCH + bc) = cb[p];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        // 16-lane group h reads k rows 8h + (j/4) (+4), columns 16t + 4*(j%4)
        const uint16_t* p = my + (8 * h + (j >> 2)) * SK_BPITCH + 16 * t + 4 * (j & 3);
        const v8 bv = cat4<v8>(lds_read_tr16(p), lds_read_tr16(p + 4 * SK_BPITCH));
        acc[t] = MT::mma(av, bv, acc[t]);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
  // lane holds column 16t + lane%16, rows 4*(lane/16) + i
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][4 * (lane >> 4) + i][16 * t + (lane & 15)] = acc[t][i];
  __syncthreads();
  constexpr int PER = 16 * SK_NT / (64 * SK_WAVES);  // outputs per thread
  float v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int o = threadIdx.x + i * 64 * SK_WAVES, r = o / SK_NT, c = o % SK_NT;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < SK_WAVES; ++w) s += red[w][r][c];
    v[i] = s;
  }
  if (nsplit > 1) {
    // the strip's tiles meet in the workspace: sc0 sc1 stores (written through), a wait for
    // them before the arrival, sc0 sc1 loads (missing every cache) after it; the sum runs in
    // split order
    const __amdgpu_buffer_rsrc_t rp =
        __builtin_amdgcn_make_buffer_rsrc(part, (short)0, 0x7fffffff, RSRC_WORD3);
#pragma unroll
    for (int i = 0; i < PER; ++i)
      __builtin_amdgcn_raw_buffer_store_b32(
          __builtin_bit_cast(uint32_t, v[i]), rp,
          (int)((blockIdx.x * SS_PART + threadIdx.x + i * 64 * SK_WAVES) * 4), 0, CP_SC01);
    __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0): the tile has been written
    __syncthreads();
    if (threadIdx.x == 0)
      last_arrival = atomicAdd(&arrivals[strip], 1u) == (unsigned)(nsplit - 1);
    __syncthreads();
    if (!last_arrival) return;
    float t[PER] = {};
    for (int sp = 0; sp < nsplit; ++sp) {  // uniform
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        float x = v[i];
        if (sp != split)
          x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
              rp, (int)(((sp * nstrips + strip) * SS_PART + threadIdx.x + i * 64 * SK_WAVES) * 4),
              0, CP_SC01));
        t[i] += x;
      }
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = t[i];
    if (threadIdx.x == 0) atomicExch(&arrivals[strip], 0u);
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int o = threadIdx.x + i * 64 * SK_WAVES, r = o / SK_NT, c = o % SK_NT;
    if (r < M && n0 + c < N) store_out<OUT>(C, (int64_t)r * N + n0 + c, v[i]);
  }
}

// ------------------------------------------------------------------------------------------------
// Split skinny GEMM (M <= 16, row-major B): the preferred form of the M <= 16 stream. B is read
// in 256-byte row segments (a 128-column strip per workgroup), and the k range is split over
// `nsplit` workgroups per strip so that about one workgroup runs per CU. Measured on the bare
// read pattern of a 4096 x 14336 fp16 B: 128-byte segments over all of K stream at 5.7 TB/s,
// 256-byte segments over half of K at 6.3 TB/s, and a workgroup per CU is needed (one CU alone
// streams about 38 GB/s). Within a workgroup the 8 waves take interleaved 16-row blocks (16 x
// 128 halves = 4 KB, one block in flight per wave), each one v_mfma_f32_16x16x16 per 16 columns.
// The workgroup's part of A (16 rows x at most 2048 k) is staged in LDS once, after each wave's
// first two B blocks are requested: per-block A fragments read from the cache were measured to
// cost 2.5 us of 24 at 16 x 14336 x 4096.
//
// The nsplit partial 16 x 128 tiles of a strip meet in a workspace: every workgroup stores its
// tile and counts itself in with an atomic on the strip's arrival counter; the last to arrive
// adds the tiles in split order (the result does not depend on arrival order), writes C and
// resets the counter to zero. The workspace is a file-scope device array with SS_SLOTS slots;
// each stream that runs this kernel on a device owns one slot, so calls that overlap are on
// different streams and never share a slot. A further stream takes gemm_skinny. A HIP graph
// keeps the slot of the stream it was captured on.

template <bool BF16>
struct mfma16k16_t;
template <>
struct mfma16k16_t<false> {
  static TLM_DEV f32x4 mma(u32x2 a, u32x2 b, f32x4 c) {
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
};
template <>
struct mfma16k16_t<true> {
  static TLM_DEV f32x4 mma(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                     __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
  }
};

template <bool BF16, int OUT>
__global__ __launch_bounds__(64 * SS_WAVES) void gemm_skinny_split(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, void* __restrict__ C, int M,
    int N, int K, int nsplit, float* __restrict__ part, unsigned* __restrict__ arrivals) {
  using MT = mfma16k16_t<BF16>;
  constexpr int AL = SS_AMAX_K * 16 * 2;
  constexpr int WB = SS_BK * SS_NT * 2;
  constexpr int LDS = AL + SS_WAVES * WB;
  static_assert(LDS >= SS_WAVES * SS_NT * 16 * 4 + 4, "reduction and flag alias the LDS");
  __shared__ __attribute__((aligned(16))) uint8_t smem[LDS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, j = lane & 15;
  const int nstrips = (N + SS_NT - 1) / SS_NT;
  const int strip = blockIdx.x % nstrips, split = blockIdx.x / nstrips;
  const int n0 = strip * SS_NT;
  const int KB = (K + SS_BK - 1) / SS_BK;
  const int kb_lo = (int)((int64_t)split * KB / nsplit);
  const int nbk = (int)((int64_t)(split + 1) * KB / nsplit) - kb_lo;  // <= SS_AMAX_K / SS_BK

  // B rows past K read as zero (past the descriptor's end), and so does a block index of KB,
  // which a wave with no block left loads; the columns past N of a ragged last strip hold
  // whatever follows and only reach output columns that are not stored.
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)B, (short)0, (int)((int64_t)K * N * 2), RSRC_WORD3);
  const int boff = g * N * 2 + (n0 + 8 * j) * 2;  // row 4p + lane/16, 16-byte chunk lane%16
  auto load = [&](u32x4 (&rb)[4], int kb) {
    const int k0 = kb * SS_BK;
#pragma unroll
    for (int p = 0; p < 4; ++p)
      rb[p] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rsb, boff + (k0 + 4 * p) * N * 2, 0, CP_NT));
  };
  // the wave's first two blocks are requested before A, so that B keeps streaming while A
  // is staged; after that one block is in flight per wave
  u32x4 rb0[4], rn[4];
  load(rb0, wave < nbk ? kb_lo + wave : KB);
  load(rn, wave + SS_WAVES < nbk ? kb_lo + wave + SS_WAVES : KB);

  // A columns 16 kb_lo .. as 16 rows of SS_AMAX_K halves, 16-byte chunk c of row m stored at
  // c ^ m: row-contiguous 1 KB loads and LDS writes, and the fragment reads of 16 rows x one
  // chunk are free of bank conflicts. The fragment of local block b (row lane%16, k 4g .. + 3)
  // is in chunk 2b + g/2 at byte 8 (g%2). Rows past M and k past K read as zero.
  constexpr int AROW = SS_AMAX_K * 2;
  {
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
        (void*)A, (short)0, (int)((int64_t)M * K * 2), RSRC_WORD3);
    constexpr int NA = SS_AMAX_K * 2 / (64 * SS_WAVES);
    const int kc0 = 2 * kb_lo, ncw = 2 * nbk, kc_end = K / 8;
    u32x4 t[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int q = i * 64 * SS_WAVES + tid, m = q / (AROW / 16), c = q % (AROW / 16);
      const int off = (m < M && c < ncw && kc0 + c < kc_end) ? (m * K + 8 * (kc0 + c)) * 2
                                                              : 0x7ffffff0;
      t[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsa, off, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int q = i * 64 * SS_WAVES + tid, m = q / (AROW / 16), c = q % (AROW / 16);
      if (c < ncw) *(u32x4*)(smem + AROW * m + 16 * (c ^ m)) = t[i];
    }
  }
  __syncthreads();

  // B staging of the wave: 16 rows of 256 bytes, 16-byte chunk c of row r stored at
  // c ^ 2 (r % 8), so that the transposed reads (4 rows x 32 bytes per 16 lanes) are free of
  // bank conflicts. Tile t: 16-lane group g reads k rows 4g + j/4, columns 16t + 4 (j%4) ..
  uint8_t* const my = smem + AL + wave * WB;
  int wr[4], rd[8];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int r = 4 * p + g;
    wr[p] = 256 * r + 16 * (j ^ (2 * (r & 7)));
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int r = 4 * g + (j >> 2), c = 2 * t + ((j & 3) >> 1);
    rd[t] = 256 * r + 16 * (c ^ (2 * (r & 7))) + 8 * (j & 1);
  }
  const uint8_t* const a_row = smem + AROW * j + 8 * (g & 1);

  f32x4 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f32x4{};
  auto process = [&](const u32x4 (&cb)[4], int b) {
    const u32x2 av = *(const u32x2*)(a_row + 16 * ((2 * b + (g >> 1)) ^ j));
#pragma unroll
    for (int p = 0; p < 4; ++p) *(u32x4*)(my + wr[p]) = cb[p];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int t = 0; t < 8; ++t)
      acc[t] = MT::mma(av, __builtin_bit_cast(u32x2, lds_read_tr16((const uint16_t*)(my + rd[t]))),
                       acc[t]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  if (wave < nbk) process(rb0, wave);
  for (int b = wave + SS_WAVES; b < nbk; b += SS_WAVES) {
    u32x4 cb[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) cb[p] = rn[p];
    load(rn, b + SS_WAVES < nbk ? kb_lo + b + SS_WAVES : KB);
    process(cb, b);
  }
  __syncthreads();  // every wave is done with A and its staging before the reduction reuses them

  // The 8 waves' tiles are summed through LDS as [wave][column][16 rows]: a lane's accumulator
  // (column 16t + lane%16, rows 4 (lane/16) .. + 3) is one 16-byte write, and a thread's share
  // of the sum (column tid/4, rows 4 (tid%4) .. + 3) one 16-byte read per wave.
  f32x4* const red = (f32x4*)smem;
#pragma unroll
  for (int t = 0; t < 8; ++t) red[(wave * SS_NT + 16 * t + j) * 4 + g] = acc[t];
  __syncthreads();
  const int ocol = tid >> 2, orow = 4 * (tid & 3);
  f32x4 v = red[tid];
#pragma unroll
  for (int w = 1; w < SS_WAVES; ++w) v += red[w * SS_NT * 4 + tid];
  if (nsplit > 1) {
    // The tiles go to memory and come back with sc0 sc1 (write-through stores, loads that miss
    // in every cache), so the exchange needs no cache write-back or invalidation: a wait for the
    // stores before the arrival, and the loads issued after it.
    st_cp<CP_SC01>(part, (blockIdx.x * SS_PART + 4 * tid) * 4, __builtin_bit_cast(u32x4, v));
    __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0): the tile has been written
    unsigned* const last = (unsigned*)(smem + LDS - 4);
    __syncthreads();
    if (tid == 0) *last = atomicAdd(&arrivals[strip], 1u) == (unsigned)(nsplit - 1);
    __syncthreads();
    if (!*last) return;
    // every other tile requested before any is added (one memory latency, not one per split;
    // nsplit and split are uniform, so the tests are scalar branches); the sum runs in split
    // order
    f32x4 pt[SS_MAX_SPLIT];
#pragma unroll
    for (int sp = 0; sp < SS_MAX_SPLIT; ++sp) {
      pt[sp] = v;
      if (sp < nsplit && sp != split)
        pt[sp] = __builtin_bit_cast(
            f32x4, ld_cp<CP_SC01>(part, ((sp * nstrips + strip) * SS_PART + 4 * tid) * 4));
    }
    f32x4 tot = {};
#pragma unroll
    for (int sp = 0; sp < SS_MAX_SPLIT; ++sp)
      if (sp < nsplit) tot += pt[sp];
    v = tot;
    if (tid == 0) atomicExch(&arrivals[strip], 0u);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (orow + i < M && n0 + ocol < N) store_out<OUT>(C, (int64_t)(orow + i) * N + n0 + ocol, v[i]);
}

// Generic fallback for shapes the vector kernels cannot take (K or N not a multiple of 8,
// unaligned pointers): one thread per output, fp32 accumulation in k order.
template <bool BF16, bool TRANS_B, int OUT>
__global__ __launch_bounds__(256) void gemm_generic(const uint16_t* __restrict__ A,
                                                    const uint16_t* __restrict__ B,
                                                    void* __restrict__ C, int M, int N, int K) {
  using H = h16<BF16>;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int m = (int)(idx / N), n = (int)(idx % N);
  float s = 0.f;
  for (int k = 0; k < K; ++k) {
    const float a = H::to_f32(A[(int64_t)m * K + k]);
    const float b = TRANS_B ? H::to_f32(B[(int64_t)n * K + k]) : H::to_f32(B[(int64_t)k * N + n]);
    s = fmaf(a, b, s);
  }
  store_out<OUT>(C, idx, s);
}

}  // namespace

// Workspace of gemm_skinny_split, one instance per GPU (a device that loads this code object
// holds its own copy until the process ends; 16 MB): SS_SLOTS slots of partial tiles and arrival
// counters. The counters start at zero and every call leaves them at zero. In host code the names
// only identify the symbols; the device addresses come from hipGetSymbolAddress.
static __device__ __align__(256) float ss_partials[SS_SLOTS][SS_MAX_WG][SS_PART];
static __device__ __align__(256) unsigned ss_arrivals[SS_SLOTS][SS_MAX_WG];

namespace {

constexpr int kSsDevices = 64;
struct SsDevice {
  std::once_flag once;
  hipError_t err = hipSuccess;
  float* part = nullptr;
  unsigned* arrivals = nullptr;
  bool used[SS_SLOTS] = {};
  hipStream_t owner[SS_SLOTS] = {};
};
SsDevice g_ss[kSsDevices];
std::mutex g_ss_mu;

// The workspace slot of stream `s` on the current device: the one it owns, else a free one that
// it then owns. False when every slot is owned by another stream (or the lookup failed), and the
// caller takes gemm_skinny.
bool ss_slot(hipStream_t s, float** part, unsigned** arrivals) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kSsDevices) return false;
  SsDevice& d = g_ss[dev];
  std::call_once(d.once, [&d]() {
    void* p = nullptr;
    void* q = nullptr;
    d.err = hipGetSymbolAddress(&p, HIP_SYMBOL(ss_partials));
    if (d.err == hipSuccess) d.err = hipGetSymbolAddress(&q, HIP_SYMBOL(ss_arrivals));
    d.part = (float*)p;
    d.arrivals = (unsigned*)q;
  });
  if (d.err != hipSuccess) return false;
  std::lock_guard<std::mutex> lk(g_ss_mu);
  int slot = -1;
  for (int i = 0; i < SS_SLOTS && slot < 0; ++i)
    if (d.used[i] && d.owner[i] == s) slot = i;
  for (int i = 0; i < SS_SLOTS && slot < 0; ++i)
    if (!d.used[i]) {
      d.used[i] = true;
      d.owner[i] = s;
      slot = i;
    }
  if (slot < 0) return false;
  *part = d.part + (size_t)slot * SS_MAX_WG * SS_PART;
  *arrivals = d.arrivals + (size_t)slot * SS_MAX_WG;
  return true;
}

// Split count of gemm_skinny_split for N x K (0: the shape does not fit it): about one
// workgroup per CU without a second round, at least 16 blocks (256 k) and at most SS_AMAX_K of
// k per workgroup.
int ss_nsplit(int N, int K) {
  const int nstrips = (N + SS_NT - 1) / SS_NT;
  const int KB = (K + SS_BK - 1) / SS_BK;
  int ns = std::max(1, std::min(SS_MAX_SPLIT, 256 / nstrips));
  ns = std::min(ns, std::max(1, KB / 16));
  ns = std::max(ns, (KB + SS_AMAX_K / SS_BK - 1) / (SS_AMAX_K / SS_BK));
  if (ns > SS_MAX_SPLIT || (ns > 1 && (int64_t)nstrips * ns > SS_MAX_WG)) return 0;
  return ns;
}

// Split count of gemm_skinny for B^T (1: no split): about one workgroup per CU when the 64-column
// strips are fewer, at least 8 blocks (256 k) per workgroup.
int sk_nsplit(int N, int K) {
  const int nstrips = (N + SK_NT - 1) / SK_NT;
  const int KB = (K + SK_BK - 1) / SK_BK;
  int ns = std::max(1, std::min(SS_MAX_SPLIT, 256 / nstrips));
  ns = std::min(ns, std::max(1, KB / 8));
  return (int64_t)nstrips * ns > SS_MAX_WG ? 1 : ns;
}

template <bool BF16, bool TRANS_B, int OUT>
int launch(const void* A, const void* B, void* C, int M, int N, int K, hipStream_t s) {
  const bool vec = tlm_aligned(A, 16) && tlm_aligned(B, 16) && K % 8 == 0 &&
                   (TRANS_B || N % 8 == 0);
  int ns = 0;
  float* part = nullptr;
  unsigned* arrivals = nullptr;
  if (vec && M <= 16 && !TRANS_B && K > 0 && (int64_t)(K + 2 * SS_BK) * N * 2 < 0x7ffffff0)
    ns = ss_nsplit(N, K);
  if (ns > 1 && !ss_slot(s, &part, &arrivals)) ns = 0;
  if (ns > 0) {
    const int nstrips = (N + SS_NT - 1) / SS_NT;
    gemm_skinny_split<BF16, OUT><<<(unsigned)(nstrips * ns), 64 * SS_WAVES, 0, s>>>(
        (const uint16_t*)A, (const uint16_t*)B, C, M, N, K, ns, part, arrivals);
  } else if (vec && M <= 16) {
    int nk = TRANS_B ? sk_nsplit(N, K) : 1;
    if (nk > 1 && !ss_slot(s, &part, &arrivals)) nk = 1;
    gemm_skinny<BF16, TRANS_B, OUT><<<(unsigned)((N + SK_NT - 1) / SK_NT * nk), 64 * SK_WAVES, 0,
                                      s>>>((const uint16_t*)A, (const uint16_t*)B, C, M, N, K, nk,
                                           part, arrivals);
  } else if (vec && (int64_t)BM * K * 2 < 0x7ffffff0 &&
             (TRANS_B ? (int64_t)BN * K * 2 : (int64_t)BK * N * 2) < 0x7ffffff0) {
    // the LDS-DMA offsets of a 256-row panel (or a 64-row k-tile of row-major B) are 32-bit
    // byte offsets below the descriptor's num_records; larger shapes take gemm_generic
    const int64_t tiles = (int64_t)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    gemm_256x256<BF16, TRANS_B, OUT><<<(unsigned)tiles, NTHREADS, 0, s>>>(
        (const uint16_t*)A, (const uint16_t*)B, C, M, N, K);
  } else {
    const int64_t n = (int64_t)M * N;
    gemm_generic<BF16, TRANS_B, OUT><<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
        (const uint16_t*)A, (const uint16_t*)B, C, M, N, K);
  }
  TLM_LAUNCH_CHECK("tlm_gemm");
  return TLM_OK;
}

template <bool BF16, bool TRANS_B>
int by_out(const void* A, const void* B, void* C, int M, int N, int K, int out, hipStream_t s) {
  switch (out) {
    case TLM_F16: return launch<BF16, TRANS_B, TLM_F16>(A, B, C, M, N, K, s);
    case TLM_BF16: return launch<BF16, TRANS_B, TLM_BF16>(A, B, C, M, N, K, s);
    default: return launch<BF16, TRANS_B, TLM_F32>(A, B, C, M, N, K, s);
  }
}

}  // namespace

extern "C" int tlm_gemm(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                        int in_dtype, int out_dtype, int trans_b, void* stream) {
  if (!A || !B || !C) {
    tlm_set_error("tlm_gemm: null pointer argument");
    return TLM_EINVAL;
  }
  if (M < 0 || N < 0 || K < 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX ||
      M * N > ((int64_t)1 << 40)) {
    tlm_set_error("tlm_gemm: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                  (long long)K);
    return TLM_EINVAL;
  }
  if (trans_b != 0 && trans_b != 1) {
    tlm_set_error("tlm_gemm: trans_b must be 0 or 1");
    return TLM_EINVAL;
  }
  if (in_dtype != TLM_F16 && in_dtype != TLM_BF16) {
    tlm_set_error("tlm_gemm: in_dtype %d unsupported (F16 or BF16)", in_dtype);
    return TLM_EUNSUPPORTED;
  }
  if (out_dtype != TLM_F16 && out_dtype != TLM_BF16 && out_dtype != TLM_F32) {
    tlm_set_error("tlm_gemm: out_dtype %d unsupported", out_dtype);
    return TLM_EUNSUPPORTED;
  }
  if (!tlm_aligned(A, 2) || !tlm_aligned(B, 2) || !tlm_aligned(C, out_dtype == TLM_F32 ? 4 : 2)) {
    tlm_set_error("tlm_gemm: misaligned pointer");
    return TLM_EINVAL;
  }
  if (M == 0 || N == 0) return TLM_OK;
  hipStream_t s = (hipStream_t)stream;
  const int m = (int)M, n = (int)N, k = (int)K;
  const bool bf = in_dtype == TLM_BF16;
  if (bf)
    return trans_b ? by_out<true, true>(A, B, C, m, n, k, out_dtype, s)
                   : by_out<true, false>(A, B, C, m, n, k, out_dtype, s);
  return trans_b ? by_out<false, true>(A, B, C, m, n, k, out_dtype, s)
                 : by_out<false, false>(A, B, C, m, n, k, out_dtype, s);
}
