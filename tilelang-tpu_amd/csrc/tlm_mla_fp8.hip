// FP8 MLA paged decode, balanced over every CU, QK^T on fp8 MFMA.
//
// Reference: examples/deepseek_mla/example_mla_decode_paged.py — per (sequence, head):
//   S = Q KV^T + Q_pe K_pe^T over the sequence's tokens (page address
//   BT[b, tok / page] * page + tok % page, :147-148), scale = sm_scale * log2(e) (:12),
//   softmax in the exp2 domain, O = P KV (:150-183), partial results merged by
//   lse = log2(sum 2^(lse_s - max)) + max, O = sum O_s 2^(lse_s - lse) (:186-221).
// FP8 config: KV is OCP e4m3 with one fp32 scale: scores use (Q . K_fp8) * kv_scale and the
// output is (P . V_fp8) * kv_scale.
//
// At 128 heads the decode does ~480 flop per KV byte, above the MI355X bf16 ridge, so this kernel
// is organised around the matrix cores:
//   * work partition: the sequences' 64-token tiles are concatenated and cut into G equal ranges,
//     so every CU gets the same number of tiles whatever the length mix. A range holds pieces of
//     one or more sequences: a sequence entirely inside one range is written to the output
//     directly; the pieces of a longer one go to partial slots (bf16 O, fp32 lse; one for the
//     range's first piece, one for its last) merged by the combine kernel;
//   * workgroup = 64 heads x one range = 2 wave pairs x 32 heads. The two waves of a pair split a
//     64-token tile by tokens for S^T = K Q^T (one 32-token block each, all 576 dims) and by V
//     dims for O^T = V^T P^T (256 dims each, all 64 tokens), exchanging block maxima and the e4m3
//     P^T block through LDS: no work is duplicated and each wave holds only 128 O accumulators;
//   * Q^T stays in VGPRs for the whole piece, split per head into two e4m3 terms
//     q / s = hi + lo (s a power of two putting max|q| at <= 448), which keeps bf16-level accuracy
//     while S^T runs on v_mfma_f32_32x32x64_f8f6f4 straight from the fp8 cache bytes (2 MFMAs per
//     64 dims: the cost of one bf16 MFMA and no K conversion);
//   * O^T = V^T P^T on the MX-scaled fp8 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4): V^T comes
//     straight from the row-major fp8 tile through ds_read_b64_tr_b8 (8 tokens of one dim per
//     lane); P^T is rounded once to e4m3 on a power-of-two scale per (head, 32-token block),
//     passed to the MFMA as its E8M0 block scale (one e4m3 term: relative RMS error ~1.3% of the
//     output against the exact softmax, against ~0.2% for two terms at one more MFMA per dim
//     block). K rows are fed to the S^T MFMA in the order tau (bits 2 and 3 of the row index
//     swapped) so S^T accumulator element i of lane l is token 16(i/8) + 8(l/32) + i%8, the
//     order of the P^T blocks exchanged through LDS;
//   * softmax without accumulator rescaling: a segment fixes its reference max m from its first
//     tile and accumulates 2^(x - m); only when a tile's max exceeds m by more than 64 (log2
//     units) does the segment end (its normalised partial is merged into a scratch slot) and a new
//     one start at that tile. fp32 holds 2^64 * 448 * 2^31 without overflow, so the result equals
//     the rescaling online softmax while the O accumulators are only ever touched by MFMAs;
//   * KV tiles (64 tokens x 576 bytes) stream into a 3-stage LDS ring with buffer_load ... lds
//     (16 bytes per lane, no VGPR round trip); each tile's buffer descriptor bounds the rows to
//     the sequence's valid tokens and to the KV pool, so rows past either read as zeros (never
//     stale NaN bytes); an explicit vmcnt wait plus s_barrier hands a stage over;
//   * LDS layout per stage: latent rows of 512 B then rope rows of 64 B, 16-byte chunks XOR-
//     swizzled so that the row reads of S^T (ds_read_b128) and the transposed reads of V^T
//     (ds_read_b64_tr_b8) are both bank-conflict free.
#include "tlm_common.h"

#include <algorithm>
#include <type_traits>

namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int F8_DV = 512, F8_DPE = 64;
constexpr int F8_TILE = 64;                          // tokens per ring stage
constexpr int F8_LAT = F8_TILE * F8_DV;              // latent bytes per stage
constexpr int F8_STAGE = F8_LAT + F8_TILE * F8_DPE;  // + rope bytes
constexpr int F8_NSTAGE = 3;
constexpr int F8_HEADS = 64;                         // heads per workgroup (2 pairs x 32)
constexpr int F8_LOADS = 9;                          // LDS-DMA loads per thread per stage
constexpr int F8_SLOTS = 3;                          // first piece, last piece, segment scratch
constexpr float F8_RESET = 64.f;                     // log2 headroom of a segment's reference
constexpr int F8_RSRC_WORD3 = 0x00020000;            // raw buffer, 32-bit data format
constexpr int F8_WAVE_F4 = 8 * 4 * 64;               // 4-element groups per wave in a partial slot
constexpr int F8_QREG = 4;                           // Q k-steps held in VGPRs; the rest in LDS
#ifndef F8_DMA_STEPS
#define F8_DMA_STEPS 3
#endif
// The refill of the ring (F8_LOADS LDS-DMA instructions per thread) is spread over the first
// F8_DMA_STEPS k-steps of the S^T MFMAs, so the tile two ahead is requested early in the step.
constexpr int F8_DMA_PER_STEP = (F8_LOADS + F8_DMA_STEPS - 1) / F8_DMA_STEPS;

// swizzled 16-byte chunk index of latent row r / rope row r
TLM_DEV int swz_lat(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }
TLM_DEV int swz_rope(int r) { return (((r >> 2) & 1) << 1) | ((r >> 3) & 1); }
// K-row order fed to the S^T MFMA (bits 2 and 3 swapped)
TLM_DEV int tau(int x) { return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1); }

TLM_DEV void wait_vm(int n) {  // s_waitcnt vmcnt(n), other counters untouched
  if (n == 0)
    __builtin_amdgcn_s_waitcnt(0x3f70);
  else
    __builtin_amdgcn_s_waitcnt(0x3f70 | F8_LOADS);
}

// Workgroup barrier that leaves the LDS-DMA loads of the ring in flight: waits for this wave's
// LDS (and scalar) accesses only, so its LDS writes are visible to the other waves afterwards.
TLM_DEV void wg_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt untouched
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Read-only table entry through the constant address space: a uniform address then becomes a
// scalar load (s_load), which neither uses VGPRs nor counts against the vmcnt ring accounting.
template <class T>
TLM_DEV T ldc(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

TLM_DEV void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// LDS reads of the ring issued as inline asm. Compiler-generated reads may be made to wait
// (vmcnt(0)) for every outstanding LDS-DMA load, including the prefetch of the next stages, when
// the compiler cannot prove they touch another stage. The caller waits with lds_wait() before
// using the result.
TLM_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
TLM_DEV i32x2 lds_tr8(const uint8_t* p) {
  i32x2 r;
  asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(r) : "v"(lds_addr(p)) : "memory");
  return r;
}
TLM_DEV i32x4 lds_b128(const void* p) {
  i32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(lds_addr(p)) : "memory");
  return r;
}
TLM_DEV i32x8 lds_2xb128(const void* p0, const void* p1) {
  const i32x4 a = lds_b128(p0), b = lds_b128(p1);
  return i32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}
// LDS write issued as inline asm, for the same reason (a compiler-generated write may be made to
// wait for the ring's LDS-DMA loads); wg_barrier() waits for it (lgkmcnt(0)) before publishing.
TLM_DEV void lds_write_b64(void* p, u32x2 v) {
  asm volatile("ds_write_b64 %0, %1" : : "v"(lds_addr(p)), "v"(v) : "memory");
}
// s_waitcnt lgkmcnt(0) that also orders the uses of the given asm-loaded operands after it
TLM_DEV void lds_wait(i32x8& a) { asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a) : : "memory"); }
// s_waitcnt lgkmcnt(n): all but the n most recent LDS accesses of this wave have completed (LDS
// accesses complete in order; no scalar loads may be outstanding). n is a compile-time constant
// after unrolling.
TLM_DEV void lgkm_wait(int n) {
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0xc07f); break;
    case 2: __builtin_amdgcn_s_waitcnt(0xc27f); break;
    case 4: __builtin_amdgcn_s_waitcnt(0xc47f); break;
    case 6: __builtin_amdgcn_s_waitcnt(0xc67f); break;
    default: __builtin_amdgcn_s_waitcnt(0xc07f); break;
  }
}
TLM_DEV void order_after(i32x8& a) { asm volatile("" : "+v"(a) : : "memory"); }
TLM_DEV void lds_wait(i32x8& a, i32x8& b) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b) : : "memory");
}
TLM_DEV void lds_wait(i32x8& a, i32x8& b, i32x8& c) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c) : : "memory");
}
// s_waitcnt lgkmcnt(0) that also orders the uses of eight asm-loaded operands after it
TLM_DEV void lds_wait(i32x2 (&r)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]),
                 "+v"(r[6]), "+v"(r[7])
               :
               : "memory");
}

TLM_DEV f32x16 mfma_fp8(i32x8 a, i32x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// A unscaled (E8M0 127 = 1), B scaled by 2^(sb - 127). Operand k order: byte j of lane half h is
// k = 32 (j / 16) + 16 h + j % 16; the scale of B's k-block kb (32 values) for column n comes
// from lane 32 kb + n.
TLM_DEV f32x16 mfma_fp8_bscaled(i32x8 a, i32x8 b, f32x16 c, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, sb);
}

// 8 e4m3 bytes -> 8 bf16 (exact)
TLM_DEV bf16x8 fp8x8_to_bf16(i32x2 v) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[0], 1.0f, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[0], 1.0f, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[1], 1.0f, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[1], 1.0f, true);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// four bf16 (two dwords) -> four floats (exact)
TLM_DEV f32x4 bf16x4_to_f32(u32x2 w) {
  return f32x4{__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u),
               __uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xffff0000u)};
}

// four floats -> four e4m3 bytes (round to nearest even)
TLM_DEV int pack_fp8x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
}

struct F8Args {
  const uint16_t* q;
  const uint16_t* q_pe;
  int64_t q_stride, qpe_stride;  // elements between (batch, head) rows
  const uint8_t* kv;
  const uint8_t* k_pe;
  int64_t kv_stride, kpe_stride, kv_rows;  // bytes between token rows; rows in the pool
  const int32_t* bt;
  const int32_t* seqlens;
  int32_t* cu;  // [B + 1] tile prefix over sequences (written by the prep kernel)
  uint8_t* qsplit;  // [B * Hq][2][576] e4m3 hi and lo terms of q / 2^qexp (written by prep)
  int32_t* qexp;    // [B * Hq] power-of-two exponent of each head's Q scale
  float* part_lse;
  u32x2* part_o;  // bf16 partial outputs, four per element
  uint16_t* out;
  int B, Hq, page, max_pages, G;
  int lmax;           // seqlens are clamped to [0, lmax = max_pages * page]
  float score_scale;  // sm_scale * log2(e)
  const float* kv_scale;
};

constexpr int F8_QROW = 2 * (F8_DV + F8_DPE);  // bytes per (sequence, head) in qsplit

// Prep kernel, one launch ahead of the decode kernel:
//   * workgroups 0 .. nq-1: one wave per (sequence, head) splits that Q row into two e4m3 terms,
//     q / 2^e = hi + lo, with 2^e the power of two that puts max|q| at <= 448; hi + lo is exact
//     for every element within 2^10 of the row maximum (a bf16/fp16 value has at most 8/11
//     significant bits and the residual of the first rounding fits e4m3's 4);
//   * workgroup nq: tile prefix over sequences, cu[b] = sum_{b' < b} ceil(L_b' / 64).
template <bool Q_BF16>
__global__ __launch_bounds__(256) void mla_fp8_prep(const F8Args a, int nq) {
  if ((int)blockIdx.x == nq) {
    __shared__ int32_t part[256];
    const int t = threadIdx.x;
    const int per = (a.B + 255) / 256;
    const int b0 = min(a.B, t * per), b1 = min(a.B, b0 + per);
    auto tiles = [&](int b) {
      const int L = max(0, min(a.seqlens[b], a.lmax));
      return (L + F8_TILE - 1) / F8_TILE;
    };
    int32_t sum = 0;
    for (int b = b0; b < b1; ++b) sum += tiles(b);
    part[t] = sum;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
      const int32_t v = t >= off ? part[t - off] : 0;
      __syncthreads();
      part[t] += v;
      __syncthreads();
    }
    int32_t run = part[t] - sum;
    for (int b = b0; b < b1; ++b) {
      a.cu[b] = run;
      run += tiles(b);
    }
    if (t == 255) a.cu[a.B] = part[255];
    return;
  }
  using H = h16<Q_BF16>;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (int64_t)a.B * a.Hq) return;
  // lane: latent dims 8 lane .. +7; lanes 0..7 also rope dims 8 lane .. +7
  const u32x4 wl = *(const u32x4*)(a.q + row * a.q_stride + 8 * lane);
  const bool has_pe = lane < 8;
  const u32x4 wp = has_pe ? *(const u32x4*)(a.q_pe + row * a.qpe_stride + 8 * lane)
                          : u32x4{0u, 0u, 0u, 0u};
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(H::lo(wl[e])), fabsf(H::hi(wl[e]))),
                             fmaxf(fabsf(H::lo(wp[e])), fabsf(H::hi(wp[e])))));
  amax = wave_max(amax);
  int ex = 0;
  if (amax > 0.f) (void)frexpf(amax * (1.0f / 448.0f), &ex);  // amax / 2^ex <= 448
  const float inv = ldexpf(1.0f, -ex);
  auto split8 = [&](u32x4 w, u32x2& hi, u32x2& lo) {
    float x[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = H::lo(w[e]) * inv;
      x[2 * e + 1] = H::hi(w[e]) * inv;
    }
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const float* y = x + 4 * h2;
      const int h = pack_fp8x4(y[0], y[1], y[2], y[3]);
      typedef float f2 __attribute__((ext_vector_type(2)));
      const f2 r01 = __builtin_amdgcn_cvt_pk_f32_fp8(h, false);
      const f2 r23 = __builtin_amdgcn_cvt_pk_f32_fp8(h, true);
      hi[h2] = (uint32_t)h;
      lo[h2] = (uint32_t)pack_fp8x4(y[0] - r01[0], y[1] - r01[1], y[2] - r23[0], y[3] - r23[1]);
    }
  };
  uint8_t* qs = a.qsplit + row * F8_QROW;
  u32x2 hi, lo;
  split8(wl, hi, lo);
  *(u32x2*)(qs + 8 * lane) = hi;
  *(u32x2*)(qs + F8_DV + F8_DPE + 8 * lane) = lo;
  if (has_pe) {
    split8(wp, hi, lo);
    *(u32x2*)(qs + F8_DV + 8 * lane) = hi;
    *(u32x2*)(qs + 2 * F8_DV + F8_DPE + 8 * lane) = lo;
  }
  if (lane == 0) a.qexp[row] = ex;
}

// Q^T operand of one head for S^T = K Q^T, from the prep kernel's split: k-step s (64 dims: 0..7
// latent, 8 rope), lane half hf holds dims 64 s + 32 hf + j at byte j. k-steps >= F8_QREG go to
// the pair's LDS copy (written by one wave of the pair). Returns the scale 2^e of the head.
TLM_DEV float load_q(const F8Args& a, int64_t row, int hf, i32x8 (&qhi)[F8_QREG],
                     i32x8 (&qlo)[F8_QREG], i32x8* qt, bool write_qt) {
  const uint8_t* qs = a.qsplit + row * F8_QROW;
#pragma unroll
  for (int k = 0; k < F8_QREG; ++k) {
    qhi[k] = *(const i32x8*)(qs + 64 * k + 32 * hf);
    qlo[k] = *(const i32x8*)(qs + F8_DV + F8_DPE + 64 * k + 32 * hf);
  }
  if (write_qt) {
#pragma unroll
    for (int k = F8_QREG; k < 9; ++k) {
      qt[(2 * (k - F8_QREG)) * 64] = *(const i32x8*)(qs + 64 * k + 32 * hf);
      qt[(2 * (k - F8_QREG) + 1) * 64] = *(const i32x8*)(qs + F8_DV + F8_DPE + 64 * k + 32 * hf);
    }
  }
  return ldexpf(1.0f, a.qexp[row]);
}

// Workgroup index -> (range, 64-head group), keeping the head groups of one range on one XCD
// (workgroup ids are dealt round-robin over the 8 XCDs) so the second read of each KV tile is an
// L2 hit.
struct F8Work {
  int g, hgi;
};
TLM_DEV F8Work f8_work(int x, int HG) {
  const int xcd = x & 7, k = x >> 3;
  return F8Work{(k / HG) * 8 + xcd, k % HG};
}

template <bool O_BF16>
__global__ __launch_bounds__(256, 1) void mla_fp8_decode(const F8Args a) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[F8_NSTAGE * F8_STAGE];
  __shared__ float xmax[2][2][32];  // [pair][token block][head]: block maxima
  __shared__ float xsum[2][2][32];  // [pair][token block][head]: block sums of P
  // P^T blocks as e4m3: [pair][token block][head][32 tokens], and the E8M0 scale of each
  // (block, head)
  __shared__ __attribute__((aligned(16))) uint8_t xq[2][2][32][32];
  __shared__ int xsc[2][2][32];
  // Q^T k-steps F8_QREG..8 of each pair: [pair][(k - F8_QREG) * 2 + hi/lo][lane]
  __shared__ __attribute__((aligned(16))) i32x8 qt[2][(9 - F8_QREG) * 2][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) index
  const int pr = wave >> 1, dh = wave & 1;  // pair (32 heads), token block / dim half
  const int hh = lane & 31, hf = lane >> 5;
  const int HG = a.Hq / F8_HEADS;
  const F8Work wk = f8_work(blockIdx.x, HG);
  if (wk.g >= a.G) return;
  const int g = wk.g, hgi = wk.hgi;
  const int head = hgi * F8_HEADS + pr * 32 + hh;
  const int64_t T = ldc(a.cu + a.B);
  const int64_t t_lo = (int64_t)g * T / a.G, t_hi = (int64_t)(g + 1) * T / a.G;
  if (t_lo >= t_hi) return;
  const float kvs = a.kv_scale ? ldc(a.kv_scale) : 1.0f;

  // first sequence with a tile in [t_lo, t_hi): largest b with cu[b] <= t_lo
  int b_first = 0;
  {
    int lo = 0, hi = a.B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (ldc(a.cu + mid) <= t_lo) lo = mid; else hi = mid - 1;
    }
    b_first = lo;
  }

  // ---- per-tile page table: lane j holds the first KV row of tile tb + j and the number of its
  // rows to load (the sequence's valid tokens that lie inside the pool; the rest read as zeros)
  int64_t tb = INT64_MIN / 2;
  uint32_t tab_lo = 0, tab_hi = 0;
  int tab_n = 0;
  auto build_table = [&](int64_t base) {
    tb = base;
    const int64_t tj = base + lane;
    tab_lo = tab_hi = 0;
    tab_n = 0;
    if (tj < t_hi) {
      int blo = 0, bhi = a.B - 1;  // largest b with cu[b] <= tj
      while (blo < bhi) {
        const int mid = (blo + bhi + 1) >> 1;
        if (a.cu[mid] <= tj) blo = mid; else bhi = mid - 1;
      }
      const int L = max(0, min(a.seqlens[blo], a.lmax));
      const int tok0 = (int)(tj - a.cu[blo]) * F8_TILE;
      const int valid = min(F8_TILE, L - tok0);
      const int64_t row0 =
          (int64_t)a.bt[(int64_t)blo * a.max_pages + tok0 / a.page] * a.page + tok0 % a.page;
      int64_t nrow = min((int64_t)valid, a.kv_rows - row0);
      if (row0 < 0 || nrow < 0) nrow = 0;
      tab_lo = (uint32_t)row0;
      tab_hi = (uint32_t)((uint64_t)row0 >> 32);
      tab_n = (int)nrow;
    }
  };
  build_table(t_lo);

  // ---- KV ring: LDS-DMA of tile t into stage (t - t_lo) % 3
  struct Dma {  // one tile's source rows (base, byte count) and ring stage
    const uint8_t* bkv;
    const uint8_t* bpe;
    int nkv, npe;
    uint8_t* st;
  };
  auto issue_setup = [&](int64_t t) {
    if (t >= tb + 64) build_table(t);
    const int j = (int)(t - tb);
    const int64_t row0 = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)tab_hi, j) << 32) |
                                   (uint32_t)__builtin_amdgcn_readlane((int)tab_lo, j));
    const int64_t nrow = __builtin_amdgcn_readlane(tab_n, j);
    const uint8_t* bkv = nrow > 0 ? a.kv + row0 * a.kv_stride : a.kv;
    const uint8_t* bpe = nrow > 0 ? a.k_pe + row0 * a.kpe_stride : a.k_pe;
    return Dma{bkv, bpe, (int)(nrow * a.kv_stride), (int)(nrow * a.kpe_stride),
               ring + (int)((t - t_lo) % F8_NSTAGE) * F8_STAGE};
  };
  // LDS-DMA instruction k (0..8) of this thread for a tile: 0..7 latent, 8 rope
  auto issue_dma = [&](const Dma& d, int k) {
    int ln = lane;
    asm volatile("" : "+v"(ln));  // offsets recomputed per use, not hoisted into live registers
    if (k < 8) {  // latent: 2 rows x 32 chunks per wave-instruction
      const int r = 2 * (8 * wave + k) + (ln >> 5);
      const int off = r * (int)a.kv_stride + 16 * ((ln & 31) ^ swz_lat(r));
      const __amdgpu_buffer_rsrc_t rk =
          __builtin_amdgcn_make_buffer_rsrc((void*)d.bkv, (short)0, d.nkv, F8_RSRC_WORD3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(d.st + (8 * wave + k) * 1024), 16,
                                               off, 0, 0, 0);
    } else {  // rope: 16 rows x 4 chunks per wave-instruction
      const int r = 16 * wave + (ln >> 2);
      const int off = r * (int)a.kpe_stride + 16 * ((ln & 3) ^ swz_rope(r));
      const __amdgpu_buffer_rsrc_t rp =
          __builtin_amdgcn_make_buffer_rsrc((void*)d.bpe, (short)0, d.npe, F8_RSRC_WORD3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, (lds_void*)(d.st + F8_LAT + wave * 1024), 16,
                                               off, 0, 0, 0);
    }
  };
  auto issue = [&](int64_t t) {
    const Dma d = issue_setup(t);
#pragma unroll
    for (int k = 0; k < F8_LOADS; ++k) issue_dma(d, k);
  };
  issue(t_lo);
  if (t_lo + 1 < t_hi) issue(t_lo + 1);

  // ---- per-lane LDS read offsets
  const int th = tau(hh);                  // K row of this lane within its 32-token block
  const int fk = (2 * hf) ^ swz_lat(th);   // latent chunk of k-step s: (4 s) ^ fk
  const int fr = (2 * hf) ^ swz_rope(th);  // rope chunks: fr, fr ^ 1
  // V^T operand of a 32-dim block: lane (dim l % 32, half h) holds tokens 16 h + 0..15 and
  // 32 + 16 h + 0..15, read as four 8-token transposes r = 0..3 at rows
  // 16 h + 8 (r & 1) + 32 (r >> 1) + (lane % 16) / 2; the swizzle depends on r & 1 only
  const int i16 = lane & 15, gq = lane >> 4;
  int vbase[2], vx[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int vrow = 16 * (gq >> 1) + 8 * par + (i16 >> 1);
    const int vu = (gq & 1) ^ swz_lat(vrow);
    vbase[par] = vrow * F8_DV + 16 * (vu & 1) + 8 * (i16 & 1) + 256 * dh;
    vx[par] = vu >> 1;
  }

  // ---- software pipeline over the tiles of a piece: the S^T MFMAs of tile t + 1 run with the
  // softmax of tile t (and its two block exchanges) interleaved between their k-steps, then the
  // O^T MFMAs of tile t. Every wave executes the same barriers per tile (A: tile t + 1 landed,
  // B: block maxima, C: P^T blocks), whatever its own tokens or segment state.
  i32x8 qhi[F8_QREG], qlo[F8_QREG];
  int64_t t = t_lo;
  int64_t issued = t_lo + 1 < t_hi ? t_lo + 2 : t_lo + 1;  // tiles [t_lo, issued) requested
  int cb = b_first;
  int64_t cb_lo = ldc(a.cu + cb), cb_hi = ldc(a.cu + cb + 1);

  // Tile x becomes visible: this thread's loads of it have landed (only tile x + 1's may still
  // be in flight), then the workgroup barrier, after which every wave is also done with the
  // stage of tile x - 2. Returns whether tile x + 1 is to be loaded now (into that stage).
  auto visible = [&](int64_t x, Dma& dma) {
    wait_vm(issued > x + 1 ? F8_LOADS : 0);
    wg_barrier();
    if (issued == x + 1 && issued < t_hi) {
      dma = issue_setup(issued);
      ++issued;
      return true;
    }
    return false;
  };
  // S^T = K Q^T of tile x for this wave's 32 tokens (rows past the sequence read as zeros and
  // are masked later), the LDS-DMA instructions of the refill in the first k-steps (REFILL) and
  // the work hook(k) after the k-step k MFMAs. No branches inside: the k-steps form one block.
  auto qk_body = [&](int64_t x, f32x16& so, const Dma& dma, auto REFILLc, auto&& hook) {
    constexpr bool REFILL = decltype(REFILLc)::value;
    const uint8_t* st = ring + (int)((x - t_lo) % F8_NSTAGE) * F8_STAGE;
    const uint8_t* krow = st + (32 * dh + th) * F8_DV;
    const uint8_t* prow = st + F8_LAT + (32 * dh + th) * F8_DPE;
    // operands of k-step k: K (32 bytes of this lane's row) and, past F8_QREG, Q^T hi/lo
    i32x8 kop[3], qop[3][2];
    auto nreads = [](int k) { return k < F8_QREG ? 2 : 6; };  // LDS reads of k-step k
    auto kread = [&](int k) {
      kop[k % 3] = k < 8 ? lds_2xb128(krow + 16 * ((4 * k) ^ fk), krow + 16 * (((4 * k) ^ fk) ^ 1))
                         : lds_2xb128(prow + 16 * fr, prow + 16 * (fr ^ 1));
      if (k >= F8_QREG) {
        const i32x8* q = &qt[pr][2 * (k - F8_QREG)][lane];
        qop[k % 3][0] = lds_2xb128(q, (const i32x4*)q + 1);
        qop[k % 3][1] = lds_2xb128(q + 64, (const i32x4*)(q + 64) + 1);
      }
    };
    kread(0);
    kread(1);
    so = f32x16{};
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      // reads of k-step k done (later LDS accesses only make the wait stricter)
      lgkm_wait(k + 1 < 9 ? nreads(k + 1) : 0);
      order_after(kop[k % 3]);
      if (k >= F8_QREG) {
        order_after(qop[k % 3][0]);
        order_after(qop[k % 3][1]);
      }
      if (k + 2 < 9) kread(k + 2);
      if constexpr (REFILL) {
#pragma unroll
        for (int j = 0; j < F8_DMA_PER_STEP; ++j)
          if (k * F8_DMA_PER_STEP + j < F8_LOADS) issue_dma(dma, k * F8_DMA_PER_STEP + j);
      }
      so = mfma_fp8(kop[k % 3], k < F8_QREG ? qhi[k] : qop[k % 3][0], so);
      so = mfma_fp8(kop[k % 3], k < F8_QREG ? qlo[k] : qop[k % 3][1], so);
      hook(k);
      sched_fence();
    }
  };
  auto qk = [&](int64_t x, f32x16& so, bool refill, const Dma& dma, auto&& hook) {
    if (refill)
      qk_body(x, so, dma, std::true_type{}, hook);
    else
      qk_body(x, so, dma, std::false_type{}, hook);
  };

  while (t < t_hi) {  // one iteration per sequence piece
    while (t >= cb_hi) {
      ++cb;
      cb_lo = cb_hi;
      cb_hi = ldc(a.cu + cb + 1);
    }
    const int L = max(0, min(ldc(a.seqlens + cb), a.lmax));
    const int64_t qr = (int64_t)cb * a.Hq + head;
    const float ch = a.score_scale * kvs * load_q(a, qr, hf, qhi, qlo, &qt[pr][0][lane], dh == 0);
    const int64_t p_lo = t, p_hi = min(t_hi, cb_hi);
    const bool complete = p_lo == cb_lo && p_hi == cb_hi;
    const int slot = p_lo == t_lo ? 0 : 1;
    bool have_scr = false, first = true;
    float lse_scr = 0.f, mref = 0.f, lsum = 0.f;
    f32x16 oacc[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) oacc[d] = f32x16{};

    // Segment end: normalise, merge with an earlier segment (scratch slot), store this wave's
    // 256 dims: to the output for a complete sequence, else to the piece's partial slot (a cut
    // segment goes to the scratch slot)
    auto flush = [&](bool cut, float m_seg) {
      const float lse_seg = m_seg + __log2f(lsum);
      float w_seg = kvs / lsum, w_old = 0.f, lse_out = lse_seg;
      if (have_scr) {
        const float mx = fmaxf(lse_scr, lse_seg);
        const float e_old = __builtin_amdgcn_exp2f(lse_scr - mx);
        const float e_seg = __builtin_amdgcn_exp2f(lse_seg - mx);
        const float tot = e_old + e_seg;
        lse_out = mx + __log2f(tot);
        w_old = e_old / tot;
        w_seg *= e_seg / tot;
      }
      const int64_t scr_slot = (int64_t)g * F8_SLOTS + 2;
      const u32x2* scr = a.part_o + ((scr_slot * HG + hgi) * 4 + wave) * F8_WAVE_F4 + lane;
      // value of output group (dt, q4) of this wave (four consecutive dims)
      auto val = [&](int dt, int q4, auto merge) {
        f32x4 v = {oacc[dt][4 * q4], oacc[dt][4 * q4 + 1], oacc[dt][4 * q4 + 2],
                   oacc[dt][4 * q4 + 3]};
        v *= w_seg;
        if constexpr (decltype(merge)::value) v += bf16x4_to_f32(scr[(dt * 4 + q4) * 64]) * w_old;
        return v;
      };
      auto store = [&](auto merge) {
        if (cut || !complete) {
          const int64_t sb = (int64_t)g * F8_SLOTS + (cut ? 2 : slot);
          u32x2* dst = a.part_o + ((sb * HG + hgi) * 4 + wave) * F8_WAVE_F4 + lane;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              const f32x4 v = val(dt, q4, merge);
              dst[(dt * 4 + q4) * 64] = u32x2{h16<true>::pack(v[0], v[1]), h16<true>::pack(v[2], v[3])};
            }
            sched_fence();
          }
          if (dh == 0 && hf == 0) a.part_lse[sb * a.Hq + head] = lse_out;
        } else {
          using H = h16<O_BF16>;
          uint16_t* o = a.out + qr * F8_DV + 256 * dh + 4 * hf;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              const f32x4 v = val(dt, q4, merge);
              *(u32x2*)(o + 32 * dt + 8 * q4) = u32x2{H::pack(v[0], v[1]), H::pack(v[2], v[3])};
            }
            sched_fence();
          }
        }
      };
      if (have_scr)
        store(std::true_type{});
      else
        store(std::false_type{});
      wait_vm(0);  // stores retire before the ring's vmcnt accounting resumes
      if (cut) {
        have_scr = true;
        lse_scr = lse_out;
      }
    };

    // prologue: S^T of the piece's first tile
    f32x16 s;
    {
      Dma dma{};
      const bool refill = visible(t, dma);
      qk(t, s, refill, dma, [](int) {});
    }
    for (; t < p_hi; ++t) {
      const uint8_t* st = ring + (int)((t - t_lo) % F8_NSTAGE) * F8_STAGE;
      const int own = L - (int)(t - cb_lo) * F8_TILE - 32 * dh;  // this wave's valid tokens
      const bool nxt = t + 1 < p_hi;
      // softmax of tile t, in pieces placed after the k-steps of the next tile's S^T:
      //   0: block max -> LDS; 2: barrier; 3: tile max, segment check, block scale; 3..6: P^T
      //   in e4m3, 4 elements per step; 6: P^T blocks -> LDS; 7: block sums and scales -> LDS,
      //   barrier; 8: row sums, B operand
      float mb = -INFINITY, ps = 0.f, sh = 0.f, m_old = 0.f, tsum = 0.f;
      int es = 0;
      bool cut = false;  // a new segment starts at this tile (flushed before its O^T update)
      int phi4[4];
      i32x8 pbh;
      int psc = 0;
      auto hook = [&](int k) {
        if (k == 0) {
          // raw scores (the log2-domain scale ch > 0 is applied inside exp2); element i is token
          // 16 (i / 8) + 8 hf + i % 8 of the block
          if (own < 32) {  // wave-uniform: the sequence ends inside this wave's block
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int tok = 16 * (i >> 3) + 8 * hf + (i & 7);
              s[i] = tok >= own ? -INFINITY : s[i];
            }
          }
#pragma unroll
          for (int i = 0; i < 16; ++i) mb = fmaxf(mb, s[i]);
          mb = xhalf_max(mb) * ch;
          xmax[pr][dh][hh] = mb;  // both lane halves write the same value
        }
        if (k == 2) wg_barrier();
        if (k == 3) {
          const float mt = fmaxf(mb, xmax[pr][dh ^ 1][hh]);  // tile max of the head
          // a tile whose max exceeds the reference by more than the headroom ends the segment;
          // P of this tile then uses the new reference and the old segment is flushed after the
          // S^T k-steps (wave-uniform decision, no branch here)
          cut = !first && __ballot(mt > mref + F8_RESET) != 0;
          m_old = mref;
          mref = (first || cut) ? mt : mref;
          first = false;
          // P^T of this wave's block in e4m3 on a per-head power-of-two scale 2^es (es =
          // exponent of the block's largest P minus 8, so scaled values are below 256), folded
          // into the exp2 argument. The row sums add the rounded P, so the weights applied to V
          // sum to one (a one-token sequence returns its V row exactly) and the largest P of a
          // segment, 2^0, is exact
          int e2 = 0;
          (void)frexpf(__builtin_amdgcn_exp2f(mb - mref), &e2);
          es = mb == -INFINITY ? 0 : max(-127, min(127, e2 - 8));
          sh = -(mref + (float)es);
        }
        if (k >= 3 && k <= 6) {
          const int q4 = k - 3;
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = __builtin_amdgcn_exp2f(fmaf(s[4 * q4 + e], ch, sh));
          phi4[q4] = pack_fp8x4(y[0], y[1], y[2], y[3]);
          typedef float f2 __attribute__((ext_vector_type(2)));
          const f2 r01 = __builtin_amdgcn_cvt_pk_f32_fp8(phi4[q4], false);
          const f2 r23 = __builtin_amdgcn_cvt_pk_f32_fp8(phi4[q4], true);
          ps += (r01[0] + r01[1]) + (r23[0] + r23[1]);
        }
        if (k == 6) {
          // element i is token 16 (i / 8) + 8 hf + i % 8 of the block
          uint8_t* rh = &xq[pr][dh][hh][8 * hf];
          lds_write_b64(rh, u32x2{(uint32_t)phi4[0], (uint32_t)phi4[1]});
          lds_write_b64(rh + 16, u32x2{(uint32_t)phi4[2], (uint32_t)phi4[3]});
        }
        if (k == 7) {
          ps = xhalf_sum(ldexpf(ps, es));
          xsum[pr][dh][hh] = ps;  // both lane halves write the same values
          xsc[pr][dh][hh] = es + 127;
          wg_barrier();
        }
        if (k == 8) {
          tsum = dh == 0 ? ps + xsum[pr][1][hh] : xsum[pr][0][hh] + ps;
          // B operand: lane (head hh, half hf) holds tokens 16 hf + 0..15 of both blocks; its
          // scale is that of block hf
          pbh = lds_2xb128(&xq[pr][0][hh][16 * hf], &xq[pr][1][hh][16 * hf]);
          psc = xsc[pr][hf][hh];
        }
      };
      f32x16 sn;
      if (nxt) {
        Dma dma{};
        const bool refill = visible(t + 1, dma);
        qk(t + 1, sn, refill, dma, hook);
      } else {
#pragma unroll
        for (int k = 0; k < 9; ++k) hook(k);
      }
      if (cut) {  // wave-uniform; rare
        flush(true, m_old);
#pragma unroll
        for (int d = 0; d < 8; ++d) oacc[d] = f32x16{};
        lsum = 0.f;
      }
      lsum += tsum;
      // O^T (this wave's 256 dims) += V^T P^T over the tile's 64 tokens: 8 dim blocks
      auto vread = [&](int dt) {
        i32x2 r[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          r[rr] = lds_tr8(st + vbase[rr & 1] + 32 * F8_DV * (rr >> 1) + 32 * (dt ^ vx[rr & 1]));
        return i32x8{r[0][0], r[0][1], r[1][0], r[1][1], r[2][0], r[2][1], r[3][0], r[3][1]};
      };
      i32x8 vop[2][2];
      vop[0][0] = vread(0);
      vop[0][1] = vread(1);
      lds_wait(pbh);
#pragma unroll
      for (int g2 = 0; g2 < 4; ++g2) {
        lds_wait(vop[g2 & 1][0], vop[g2 & 1][1]);
        if (g2 + 1 < 4) {
          vop[(g2 + 1) & 1][0] = vread(2 * g2 + 2);
          vop[(g2 + 1) & 1][1] = vread(2 * g2 + 3);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int dt = 2 * g2 + u;
          oacc[dt] = mfma_fp8_bscaled(vop[g2 & 1][u], pbh, oacc[dt], psc);
        }
        sched_fence();
      }
      if (nxt) s = sn;
    }
    flush(false, mref);
  }
}

// Merge the partial slots of every sequence that spans more than one range; zero-length
// sequences produce zeros. Workgroup = (sequence, 64-head group, 32-dim block of each half);
// wave w reads what decode wave w stored, in the same lane layout.
template <bool O_BF16>
__global__ __launch_bounds__(256) void mla_fp8_combine(const F8Args a) {
  const int HG = a.Hq / F8_HEADS;
  const int dt = blockIdx.x & 7;
  const int bh = blockIdx.x >> 3;
  const int hgi = bh % HG, b = bh / HG;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pr = wave >> 1, dh = wave & 1;
  const int hh = lane & 31, hf = lane >> 5;
  const int head = hgi * F8_HEADS + pr * 32 + hh;
  using H = h16<O_BF16>;
  uint16_t* o = a.out + ((int64_t)b * a.Hq + head) * F8_DV + 256 * dh + 32 * dt + 4 * hf;
  const int64_t T = a.cu[a.B], c0 = a.cu[b], c1 = a.cu[b + 1];
  if (c0 == c1) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) *(u32x2*)(o + 8 * q4) = u32x2{0u, 0u};
    return;
  }
  const int64_t G = a.G;
  const int64_t g0 = ((c0 + 1) * G - 1) / T, g1 = (c1 * G - 1) / T;
  if (g0 == g1) return;  // whole sequence inside one range: written by the decode kernel
  auto start = [&](int64_t g) { return g * T / G; };
  auto slot_of = [&](int64_t g) { return g * F8_SLOTS + ((g == g0 && c0 != start(g0)) ? 1 : 0); };
  // Online merge over the ranges in batches of F8_CMB: the lse values and partial outputs of a
  // batch are all requested before any is used, so a call waits for about one memory latency
  // per batch (a sequence spans at most a few ranges at the usual split counts).
  constexpr int F8_CMB = 8;
  float m = -INFINITY, l = 0.f;
  f32x4 acc[4] = {};
  for (int64_t gb = g0; gb <= g1; gb += F8_CMB) {
    float lv[F8_CMB];
    u32x2 pv[F8_CMB][4];
#pragma unroll
    for (int i = 0; i < F8_CMB; ++i) {
      const int64_t g = gb + i;  // wave-uniform
      lv[i] = -INFINITY;
      if (g <= g1 && start(g) != start(g + 1)) {
        const int64_t sb = slot_of(g);
        lv[i] = a.part_lse[sb * a.Hq + head];
        const u32x2* src =
            a.part_o + ((sb * HG + hgi) * 4 + wave) * F8_WAVE_F4 + dt * 4 * 64 + lane;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) pv[i][q4] = src[q4 * 64];
      } else {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) pv[i][q4] = u32x2{0u, 0u};
      }
    }
    float mb = m;
#pragma unroll
    for (int i = 0; i < F8_CMB; ++i) mb = fmaxf(mb, lv[i]);
    const float r = __builtin_amdgcn_exp2f(m - mb);  // m = -inf on the first batch: r = 0
    l *= r;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) acc[q4] *= r;
#pragma unroll
    for (int i = 0; i < F8_CMB; ++i) {
      const float w = __builtin_amdgcn_exp2f(lv[i] - mb);  // 0 for an absent range
      l += w;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) acc[q4] += bf16x4_to_f32(pv[i][q4]) * w;
    }
    m = mb;
  }
  const float inv = 1.0f / l;
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) acc[q4] *= inv;
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4)
    *(u32x2*)(o + 8 * q4) = u32x2{H::pack(acc[q4][0], acc[q4][1]), H::pack(acc[q4][2], acc[q4][3])};
}

size_t f8_align(size_t n) { return (n + 255) & ~(size_t)255; }
size_t f8_cu_bytes(int64_t B) { return f8_align((size_t)(B + 1) * 4); }
size_t f8_q_bytes(int64_t B, int64_t Hq) {
  return f8_align((size_t)B * Hq * F8_QROW) + f8_align((size_t)B * Hq * 4);
}

// ranges per call: B * num_split workgroups shared by the Hq / 64 head groups
int64_t f8_ranges(int64_t B, int64_t Hq, int num_split) {
  return std::max<int64_t>(1, B * num_split / (Hq / F8_HEADS));
}

}  // namespace

// Workspace of the fp8 path: tile prefix, Q terms, then lse (fp32) and O (bf16) partial slots
// (three 64-head x 512 slots per range and head group).
size_t tlm_mla_fp8_workspace_bytes(int64_t B, int64_t Hq, int num_split) {
  if (Hq % F8_HEADS) return 0;
  const size_t G = (size_t)f8_ranges(B, Hq, num_split);
  return f8_cu_bytes(B) + f8_q_bytes(B, Hq) +
         G * F8_SLOTS * (size_t)Hq * (F8_DV * sizeof(uint16_t) + sizeof(float));
}

// Whether the fp8 matrix-core path takes this shape (fp8 KV is checked by the caller).
bool tlm_mla_fp8_applies(int64_t B, int64_t Hq, int64_t page, int64_t max_pages,
                         int64_t kv_stride, int64_t kpe_stride) {
  const int64_t tiles_per_seq = (max_pages * page + F8_TILE - 1) / F8_TILE;
  return Hq % F8_HEADS == 0 && page % F8_TILE == 0 && kv_stride <= (1 << 24) &&
         kpe_stride <= (1 << 24) && B * tiles_per_seq <= INT32_MAX;
}

// Returns TLM_EUNSUPPORTED (launching nothing) when the shape is outside this kernel's domain.
int tlm_mla_fp8_launch(const void* q, const void* q_pe, int64_t q_stride, int64_t q_pe_stride,
                       const void* kv, const void* k_pe, int64_t kv_stride, int64_t kpe_stride,
                       int64_t kv_rows, const int32_t* block_table, const int32_t* seqlens,
                       void* o, void* ws, int64_t B, int64_t Hq, int64_t page, int64_t max_pages,
                       int num_split, float score_scale, const float* kv_scale, bool q_bf16,
                       bool o_bf16, void* stream) {
  if (!tlm_mla_fp8_applies(B, Hq, page, max_pages, kv_stride, kpe_stride))
    return TLM_EUNSUPPORTED;
  F8Args a;
  a.q = (const uint16_t*)q;
  a.q_pe = (const uint16_t*)q_pe;
  a.q_stride = q_stride;
  a.qpe_stride = q_pe_stride;
  a.kv = (const uint8_t*)kv;
  a.k_pe = (const uint8_t*)k_pe;
  a.kv_stride = kv_stride;
  a.kpe_stride = kpe_stride;
  a.kv_rows = kv_rows;
  a.bt = block_table;
  a.seqlens = seqlens;
  a.cu = (int32_t*)ws;
  const int64_t G = f8_ranges(B, Hq, num_split);
  a.qsplit = (uint8_t*)ws + f8_cu_bytes(B);
  a.qexp = (int32_t*)(a.qsplit + f8_align((size_t)B * Hq * F8_QROW));
  a.part_lse = (float*)((char*)ws + f8_cu_bytes(B) + f8_q_bytes(B, Hq));
  a.part_o = (u32x2*)(a.part_lse + G * F8_SLOTS * Hq);
  a.out = (uint16_t*)o;
  a.B = (int)B;
  a.Hq = (int)Hq;
  a.page = (int)page;
  a.max_pages = (int)max_pages;
  a.G = (int)G;
  a.lmax = (int)(max_pages * page);
  a.score_scale = score_scale;
  a.kv_scale = kv_scale;
  hipStream_t st = (hipStream_t)stream;
  const int HG = (int)(Hq / F8_HEADS);
  const int nq = (int)((B * Hq + 3) / 4);
  if (q_bf16)
    mla_fp8_prep<true><<<nq + 1, 256, 0, st>>>(a, nq);
  else
    mla_fp8_prep<false><<<nq + 1, 256, 0, st>>>(a, nq);
  TLM_LAUNCH_CHECK("tlm_mla_decode (fp8 prep)");
  const dim3 grid((unsigned)(((G + 7) / 8) * 8 * HG));
  if (o_bf16)
    mla_fp8_decode<true><<<grid, 256, 0, st>>>(a);
  else
    mla_fp8_decode<false><<<grid, 256, 0, st>>>(a);
  TLM_LAUNCH_CHECK("tlm_mla_decode (fp8 decode)");
  const dim3 cgrid((unsigned)(B * HG * 8));
  if (o_bf16) mla_fp8_combine<true><<<cgrid, 256, 0, st>>>(a);
  else mla_fp8_combine<false><<<cgrid, 256, 0, st>>>(a);
  TLM_LAUNCH_CHECK("tlm_mla_decode (fp8 combine)");
  return TLM_OK;
}
