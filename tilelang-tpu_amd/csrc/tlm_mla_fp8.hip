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
//   * two decode kernels share the partition, the Q terms, the P rounding and the combine:
//     mla_fp8_decode_w32 (Hq a multiple of 128, the config) gives a workgroup 128 heads and each
//     of its 4 waves 32 heads for the whole tile (described at the kernel); mla_fp8_decode (Hq a
//     multiple of 64 otherwise) gives a workgroup 64 heads in 8 waves (two per SIMD) = 2 head
//     blocks of 32 x 4 waves. There, for S^T = K Q^T the four waves of a head block split a
//     64-token tile into 2 token blocks x 2 halves of the 576 QK dims, and each wave keeps half
//     of its block's tokens, adding the other half's partial scores received through LDS; for
//     O^T = V^T P^T they split the 512 V dims four ways over all 64 tokens;
//   * Q^T (in VGPRs; its lo term in LDS in the 128-head kernel) is split per head into two e4m3
//     terms q / s = hi + lo (s a power of two putting max|q| at <= 448): bf16-level accuracy
//     while S^T runs on v_mfma_f32_32x32x64_f8f6f4 straight from the fp8 cache bytes (2 MFMAs per
//     64 dims: the cost of one bf16 MFMA and no K conversion; the rope dims take the hi term on
//     one dim half and the lo term on the other, so both halves run 9 MFMAs);
//   * O^T = V^T P^T on the MX-scaled fp8 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4): V^T comes
//     straight from the row-major fp8 tile through ds_read_b64_tr_b8 (8 tokens of one dim per
//     lane); P^T is rounded once to e4m3 on a power-of-two scale per (head, 32-token block),
//     passed to the MFMA as its E8M0 block scale (one e4m3 term: relative RMS error ~1.3% of the
//     output against the exact softmax, against ~0.2% for two terms at one more MFMA per dim
//     block). K rows are fed to the S^T MFMA in the order tau (bits 2 and 3 of the row index
//     swapped; bit 4 flipped on dim half 1) so that accumulator elements 0..7 of lane l are the 8
//     consecutive tokens 16 dq + 8(l/32) + 0..7 that the wave keeps, the byte order of the P^T
//     blocks exchanged through LDS;
//   * softmax without per-tile rescaling: the reference max m of a head is fixed when its
//     first block is seen and 2^(x - m) accumulates; only a block whose max exceeds m by more
//     than 64 (log2 units) moves it. fp32 holds 2^64 * 448 * 2^31 without overflow, so the result
//     equals the rescaling online softmax while the O accumulators are touched by MFMAs only. The
//     64-head kernel ends a segment there (its normalised partial merges into a scratch slot);
//     the 128-head kernel keeps whole-number references and scales what it holds by the exact
//     power of two instead;
//   * KV tiles (64 tokens x 576 bytes) stream into an LDS ring (3 stages; 2 in the 128-head
//     kernel) with buffer_load ... lds
//     (16 bytes per lane, no VGPR round trip); each tile's buffer descriptor bounds the rows to
//     the sequence's valid tokens and to the KV pool, so rows past either read as zeros (never
//     stale NaN bytes); an explicit vmcnt wait plus s_barrier hands a stage over;
//   * LDS layout per stage: latent rows of 512 B then rope rows of 64 B, 16-byte chunks XOR-
//     swizzled so that the row reads of S^T (ds_read_b128) and the transposed reads of V^T
//     (ds_read_b64_tr_b8) are both bank-conflict free;
//   * the softmax runs as short levels of independent instructions between S^T MFMAs (a wave
//     issues in order; a long dependent chain there would hold back the MFMAs), and nothing in
//     the tile loop may be spilled: a scratch reload there costs a vmcnt(0) wait on the ring's
//     in-flight LDS-DMA loads.
#include "tlm_common.h"

#include <algorithm>
#include <type_traits>
#include <utility>

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
constexpr int F8_HEADS = 64;                         // heads per workgroup (2 blocks x 32)
constexpr int F8_LAT_LOADS = 4;                      // latent LDS-DMA loads per thread per stage
constexpr int F8_PIECE_COST = 3;                    // tiles' worth of work of a piece
constexpr int F8_SLOTS = 3;
// cache policy of the KV-cache LDS-DMA loads: non-temporal (bit 1 on gfx950). The cache is read
// once per call; streaming it leaves L2 and the Infinity Cache to Q and the partial slots
// (whole call ~1-2% faster back to back, ~12% after a cache flush).
constexpr int F8_KV_NT = 2;                          // first piece, last piece, segment scratch
constexpr float F8_RESET = 64.f;                     // log2 headroom of a segment's reference
constexpr int F8_RSRC_WORD3 = 0x00020000;            // raw buffer, 32-bit data format
// cache policies (st_cp / ld_cp bits): the decode's output / partial row stores, the combine's
// partial loads and output stores
constexpr int F8_ROW_CP = CP_PLAIN;
constexpr int F8_CMB_LOAD_CP = CP_GLOBAL, F8_CMB_STORE_CP = CP_GLOBAL;

// swizzled 16-byte chunk index of latent row r / rope row r
TLM_DEV int swz_lat(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }
TLM_DEV int swz_rope(int r) { return (((r >> 2) & 1) << 1) | ((r >> 3) & 1); }
// K-row order fed to the S^T MFMA (bits 2 and 3 swapped)
TLM_DEV int tau(int x) { return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1); }

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

// f(std::integral_constant<int, i>{}) for i = 0 .. N-1, unrolled at compile time
template <typename F, int... I>
TLM_DEV void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
TLM_DEV void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// LDS accesses issued as inline asm. Compiler-generated reads may be made to wait (vmcnt(0)) for
// every outstanding LDS-DMA load, including the prefetch of the next stages, when the compiler
// cannot prove they touch another stage; asm accesses also keep the lgkmcnt accounting of the
// kernel exact. The caller waits (lgkm<N>()) and then orders the uses (order_after) itself.
TLM_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
TLM_DEV i32x2 lds_tr8(const uint8_t* p) {
  i32x2 r;
  asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(r) : "v"(lds_addr(p)) : "memory");
  return r;
}
template <int OFF>
TLM_DEV i32x2 lds_tr8_off(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  i32x2 r;
  asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}
TLM_DEV i32x4 lds_b128(const void* p) {
  i32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(lds_addr(p)) : "memory");
  return r;
}
template <int OFF>
TLM_DEV i32x4 lds_b128_off(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  i32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}
TLM_DEV i32x8 lds_2xb128(const void* p0, const void* p1) {
  const i32x4 a = lds_b128(p0), b = lds_b128(p1);
  return i32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}
TLM_DEV void lds_write_b64(void* p, u32x2 v) {
  asm volatile("ds_write_b64 %0, %1" : : "v"(lds_addr(p)), "v"(v) : "memory");
}
TLM_DEV void lds_write_b64_at(uint32_t addr, u32x2 v) {
  asm volatile("ds_write_b64 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
TLM_DEV void lds_write_b32(void* p, uint32_t v) {
  asm volatile("ds_write_b32 %0, %1" : : "v"(lds_addr(p)), "v"(v) : "memory");
}
// s_waitcnt lgkmcnt(n): all but the n most recent LDS accesses of this wave have completed (LDS
// accesses complete in order; no scalar loads may be outstanding). n is a compile-time constant
// after unrolling.
template <int N>
TLM_DEV void lgkm() {
  static_assert(N >= 0 && N < 16, "lgkmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0xc07f | (N << 8));
}
TLM_DEV void lgkm_wait(int n) {
  switch (n) {
    case 0: lgkm<0>(); break;
    case 1: lgkm<1>(); break;
    case 2: lgkm<2>(); break;
    case 3: lgkm<3>(); break;
    case 4: lgkm<4>(); break;
    case 5: lgkm<5>(); break;
    case 6: lgkm<6>(); break;
    case 7: lgkm<7>(); break;
    case 8: lgkm<8>(); break;
    case 9: lgkm<9>(); break;
    case 10: lgkm<10>(); break;
    case 11: lgkm<11>(); break;
    case 12: lgkm<12>(); break;
    default: lgkm<0>(); break;
  }
}
// makes later uses of an asm-loaded value depend on a preceding wait
TLM_DEV void order_after(i32x8& a) { asm volatile("" : "+v"(a) : : "memory"); }
TLM_DEV void order_after(i32x4& a) { asm volatile("" : "+v"(a) : : "memory"); }
TLM_DEV f32x4 as_f32x4(i32x4 v) {
  return f32x4{__int_as_float(v[0]), __int_as_float(v[1]), __int_as_float(v[2]),
               __int_as_float(v[3])};
}

TLM_DEV f32x16 mfma_fp8(i32x8 a, i32x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// The same product with its accumulator held in VGPRs, for a kernel whose AGPRs all hold other
// accumulators (the builtin's register form is chosen for the whole kernel). As inline asm it is
// outside the compiler's hazard checks, which the caller takes over: an s_nop 1 ahead of each
// MFMA covers a VALU write of an operand just before it, and xdl_settle() goes between the last
// MFMA of a chain and the first VALU read of its result (the product is 16 passes). Operands
// loaded from LDS by inline asm are waited for by the caller as with every asm load here.
TLM_DEV void mfma_fp8_v0(f32x16& d, const i32x8& a, const i32x8& b) {  // d = a b
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
}
TLM_DEV void mfma_fp8_v(f32x16& d, const i32x8& a, const i32x8& b) {  // d += a b
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}
// d = a b with b's k-blocks scaled by 2^(sb - 127) (a unscaled), accumulator in VGPRs
TLM_DEV void mfma_fp8_v0_bscaled(f32x16& d, const i32x8& a, const i32x8& b, int sb) {
  asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, 0, %3, %4 op_sel_hi:[0,0,0]"
               : "=&v"(d) : "v"(a), "v"(b), "v"(127), "v"(sb));
}
TLM_DEV void xdl_settle() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }
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
  int32_t* cu;       // [B + 1] tile prefix over sequences (written by the prep kernel)
  int32_t* vcu;      // [B + 1] cost prefix: cu plus F8_PIECE_COST per non-empty sequence before
  int32_t* range_t;  // [G + 1] first tile of each range (range g: [range_t[g], range_t[g + 1]))
  uint8_t* qsplit;  // [B * Hq][2][576] e4m3 hi and lo terms of q / 2^qexp (written by prep)
  int32_t* qexp;    // [B * Hq] power-of-two exponent of each head's Q scale
  float* part_lse;
  uint16_t* part_o;  // bf16 partial outputs [slot][head][512]
  uint16_t* out;
  int B, Hq, page, max_pages, G;
  int lmax;           // seqlens are clamped to [0, lmax = max_pages * page]
  float score_scale;  // sm_scale * log2(e)
  const float* kv_scale;
  // Split programs (glse / Output_partial written): the decode runs over B = batch * nsp
  // segments, segment v being split v % nsp of sequence v / nsp in the program's partition;
  // `out` then holds each segment's normalised rows (bf16) and seg_lse its log2 sum-exp.
  // nsp == 1, seg_lse == nullptr: the segments are the sequences.
  int nsp;
  float* seg_lse;
};

// Segment v: its sequence, first token, valid tokens and 64-token tiles (Lraw: the sequence's
// cache length). Split s of a sequence of T 64-token blocks takes T / nsp blocks, one more for
// s < T % nsp, starting after the earlier splits' blocks (example_mla_decode_paged.py:140-144
// with block_N = 64).
struct F8Seg {
  int b, start, len, ntiles;
};
TLM_DEV int f8_seq(const F8Args& a, int v) { return a.nsp == 1 ? v : v / a.nsp; }
TLM_DEV F8Seg f8_seg(const F8Args& a, int v, int Lraw) {
  const int L = max(0, min(Lraw, a.lmax));
  if (a.nsp == 1) return F8Seg{v, 0, L, (L + F8_TILE - 1) / F8_TILE};
  const int b = v / a.nsp, sp = v - b * a.nsp;
  const int tb = (L + F8_TILE - 1) / F8_TILE, bps = tb / a.nsp, rem = tb - bps * a.nsp;
  const int n = bps + (sp < rem ? 1 : 0), st = (bps * sp + min(sp, rem)) * F8_TILE;
  return F8Seg{b, st, max(0, min(n * F8_TILE, L - st)), n};
}

constexpr int F8_QROW = 2 * (F8_DV + F8_DPE);  // bytes per (sequence, head) in qsplit

// Prep kernel, one launch ahead of the decode kernel:
//   * workgroups 1 .. nq: one wave per (sequence, head) splits that Q row into two e4m3 terms,
//     q / 2^e = hi + lo, with 2^e the power of two that puts max|q| at <= 448; hi + lo is exact
//     for every element within 2^10 of the row maximum (a bf16/fp16 value has at most 8/11
//     significant bits and the residual of the first rounding fits e4m3's 4);
//   * workgroup 0 (dispatched first, so its dependent loads overlap the Q split): tile prefix
//     over sequences, cu[b] = sum_{b' < b} ceil(L_b' / 64), and the
//     ranges: the cost of a sequence is its tiles plus F8_PIECE_COST (the fixed work of a piece:
//     its Q fetch and its row flush, in tiles), the cost line [0, V) is cut into G equal ranges
//     and range g starts at the first tile at or after cost position floor(g V / G) (a range
//     starting inside a sequence's piece cost starts at its first tile). Ranges holding a
//     sequence start then get fewer tiles.
// floor / ceil of n / d for 0 <= n < 2^53, 0 < d: a double quotient corrected by integer
// products (a 64-bit integer division is a long software routine on the GPU)
TLM_DEV int64_t div_floor(int64_t n, int64_t d) {
  int64_t q = (int64_t)((double)n / (double)d);
  while (q * d > n) --q;
  while ((q + 1) * d <= n) ++q;
  return q;
}
TLM_DEV int64_t div_ceil(int64_t n, int64_t d) { return div_floor(n + d - 1, d); }

template <bool Q_BF16>
__global__ __launch_bounds__(256) void mla_fp8_prep(const F8Args a, int nq) {
  if (blockIdx.x == 0) {
    __shared__ int32_t part[256], vpart[256];
    const int t = threadIdx.x;
    const int per = (a.B + 255) / 256;
    const int b0 = min(a.B, t * per), b1 = min(a.B, b0 + per);
    auto tiles = [&](int v) { return f8_seg(a, v, a.seqlens[f8_seq(a, v)]).ntiles; };
    auto cost = [&](int n) { return n ? n + F8_PIECE_COST : 0; };
    int32_t sum = 0, vsum = 0;
    for (int b = b0; b < b1; ++b) {
      const int n = tiles(b);
      sum += n;
      vsum += cost(n);
    }
    part[t] = sum;
    vpart[t] = vsum;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
      const int32_t v = t >= off ? part[t - off] : 0, vv = t >= off ? vpart[t - off] : 0;
      __syncthreads();
      part[t] += v;
      vpart[t] += vv;
      __syncthreads();
    }
    const int64_t V = vpart[255], G = a.G;
    int32_t run = part[t] - sum, vrun = vpart[t] - vsum;
    for (int b = b0; b < b1; ++b) {
      const int n = tiles(b), vn = cost(n);
      a.cu[b] = run;
      a.vcu[b] = vrun;
      // ranges whose cost start floor(g V / G) lies in this sequence's [vrun, vrun + vn)
      if (vn > 0) {
        for (int64_t g = div_ceil(vrun * G, V); g < G; ++g) {
          const int64_t v = div_floor(g * V, G);
          if (v >= vrun + vn) break;
          a.range_t[g] = run + (int)max((int64_t)0, v - vrun - F8_PIECE_COST);
        }
      }
      run += n;
      vrun += vn;
    }
    if (t == 255) {
      a.cu[a.B] = part[255];
      a.vcu[a.B] = vpart[255];
      a.range_t[a.G] = part[255];
      if (V == 0)  // no tiles at all: every range is empty
        for (int g = 0; g < a.G; ++g) a.range_t[g] = 0;
    }
    return;
  }
  using H = h16<Q_BF16>;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)(blockIdx.x - 1) * 4 + (threadIdx.x >> 6);
  if (row >= (int64_t)(a.B / a.nsp) * a.Hq) return;
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

// Q^T operand of one head for one dim half dq of S^T = K Q^T, from the prep kernel's split. Latent
// k-step s (0..3) covers dims 256 dq + 64 s .. +63; lane half hf holds dims 32 hf .. 32 hf + 31 of
// a k-step at bytes 0..31 (the byte order of the K operand read from the ring). The rope k-step
// takes the hi term on dim half 0 and the lo term on dim half 1, so both halves run 9 MFMAs.
// Returns the head's scale 2^e.
TLM_DEV float load_q(const F8Args& a, int64_t row, int dq, int hf, i32x8 (&qhi)[4],
                     i32x8 (&qlo)[4], i32x8& qpe) {
  const uint8_t* qs = a.qsplit + row * F8_QROW;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    qhi[s] = *(const i32x8*)(qs + 256 * dq + 64 * s + 32 * hf);
    qlo[s] = *(const i32x8*)(qs + F8_DV + F8_DPE + 256 * dq + 64 * s + 32 * hf);
  }
  qpe = *(const i32x8*)(qs + dq * (F8_DV + F8_DPE) + F8_DV + 32 * hf);
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

// s_waitcnt vmcnt(N) with the other counters untouched
template <int N>
TLM_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x3f70 | (N & 15) | ((N >> 4) << 14));  // vmcnt bits 3:0 and 15:14
}

// Workgroup = 64 heads x one range, 8 waves (two per SIMD). Wave w: head block hb = w / 4 (32
// heads) and q = w % 4, with token block tq = q % 2 and dim half dq = q / 2:
//   * S^T: the wave computes the partial scores of the 32-token block tq over its half dq of the
//     576 QK dims (9 MFMAs with Q in registers), keeps tokens 16 dq .. 16 dq + 15 of the block and
//     adds the other half's partial for them, received through LDS;
//   * O^T: the wave accumulates dims 128 q .. 128 q + 127 of the head block's 32 heads over all 64
//     tokens (4 MFMAs) from the e4m3 P^T blocks that the head block's four waves publish.
// Every wave runs the same barriers per tile (A: tile t + 1 landed and the partial scores of tile
// t published, B: 16-token maxima, C: P^T blocks and sums).
template <bool O_BF16>
__global__ __launch_bounds__(512) void mla_fp8_decode(const F8Args a) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[F8_NSTAGE * F8_STAGE];
  // partial S^T exchange: [head block][token block][receiving dim half][4-element group][lane]
  __shared__ f32x4 xs[2][2][2][2][64];
  // [head block][head], component q: 16-token maxima (log2 units) / sums of the rounded P
  __shared__ f32x4 xmax[2][32];
  __shared__ f32x4 xsum[2][32];
  // P^T in e4m3: [head block][token block][16-token half][head][16 tokens]
  __shared__ __attribute__((aligned(16))) uint8_t xq[2][2][2][32][16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) index
  const int hb = wave >> 2, q = wave & 3, tq = q & 1, dq = q >> 1;
  const int hh = lane & 31, hf = lane >> 5;
  const int HG = a.Hq / F8_HEADS;
  const F8Work wk = f8_work(blockIdx.x, HG);
  if (wk.g >= a.G) return;
  const int g = wk.g, hgi = wk.hgi;
  const int head = hgi * F8_HEADS + hb * 32 + hh;
  // tile indices fit int32 (the tile prefix is int32)
  const int t_lo = ldc(a.range_t + g), t_hi = ldc(a.range_t + g + 1);
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
  int tb = INT32_MIN / 2;
  uint32_t tab_lo = 0, tab_hi = 0;
  int tab_n = 0;
  auto build_table = [&](int base) {
    tb = base;
    const int tj = base + lane;
    tab_lo = tab_hi = 0;
    tab_n = 0;
    if (tj < t_hi) {
      int blo = 0, bhi = a.B - 1;  // largest b with cu[b] <= tj
      while (blo < bhi) {
        const int mid = (blo + bhi + 1) >> 1;
        if (a.cu[mid] <= tj) blo = mid; else bhi = mid - 1;
      }
      const int L = max(0, min(a.seqlens[blo], a.lmax));
      const int tok0 = (tj - a.cu[blo]) * F8_TILE;
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

  // ---- KV ring: LDS-DMA of tile t into stage (t - t_lo) % 3; every wave loads 8 latent rows
  // (F8_LAT_LOADS instructions), waves 0..3 also 16 rope rows each
  struct Dma {  // one tile's source rows (base, byte count) and ring stage
    const uint8_t* bkv;
    const uint8_t* bpe;
    int nkv, npe;
    uint8_t* st;
  };
  auto stage = [&](int si) { return ring + si * F8_STAGE; };
  auto next_stage = [](int si) { return si == F8_NSTAGE - 1 ? 0 : si + 1; };
  int s_issue = 0;  // ring stage of the next tile to request
  auto issue_setup = [&](int t) {
    if (t >= tb + 64) build_table(t);
    const int j = t - tb;
    const int64_t row0 = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)tab_hi, j) << 32) |
                                   (uint32_t)__builtin_amdgcn_readlane((int)tab_lo, j));
    const int64_t nrow = __builtin_amdgcn_readlane(tab_n, j);
    const uint8_t* bkv = nrow > 0 ? a.kv + row0 * a.kv_stride : a.kv;
    const uint8_t* bpe = nrow > 0 ? a.k_pe + row0 * a.kpe_stride : a.k_pe;
    const Dma d{bkv, bpe, (int)(nrow * a.kv_stride), (int)(nrow * a.kpe_stride), stage(s_issue)};
    s_issue = next_stage(s_issue);
    return d;
  };
  const bool rope_loader = wave < 4;  // wave-uniform
  // LDS-DMA instruction k of this thread for a tile: 0..F8_LAT_LOADS-1 latent, then rope
  // latent instruction k of lane (c, h) = (lane % 32, lane / 32) reads row r = 8 w + 2 k + h at
  // swizzled chunk c ^ swz_lat(r) = (c ^ (2 h + (w & 1))) ^ 4 k
  const int lat_off = (2 * F8_LAT_LOADS * wave + hf) * (int)a.kv_stride;
  const int lat_x16 = 16 * (hh ^ (2 * hf + (wave & 1)));
  auto issue_dma = [&](const Dma& d, int k) {
    if (k < F8_LAT_LOADS) {  // latent: 2 rows x 32 chunks per wave-instruction
      const int ki = F8_LAT_LOADS * wave + k;
      const int off = lat_off + 2 * k * (int)a.kv_stride + (lat_x16 ^ (64 * k));
      const __amdgpu_buffer_rsrc_t rk =
          __builtin_amdgcn_make_buffer_rsrc((void*)d.bkv, (short)0, d.nkv, F8_RSRC_WORD3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(d.st + ki * 1024), 16, off, 0, 0,
                                               F8_KV_NT);
    } else {  // rope: 16 rows x 4 chunks per wave-instruction
      int ln;  // lane id computed here, not kept in a register across the tile
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
      const int r = 16 * wave + (ln >> 2);
      const int off = r * (int)a.kpe_stride + 16 * ((ln & 3) ^ swz_rope(r));
      const __amdgpu_buffer_rsrc_t rp =
          __builtin_amdgcn_make_buffer_rsrc((void*)d.bpe, (short)0, d.npe, F8_RSRC_WORD3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, (lds_void*)(d.st + F8_LAT + wave * 1024), 16,
                                               off, 0, 0, F8_KV_NT);
    }
  };
  auto issue = [&](int t) {
    const Dma d = issue_setup(t);
#pragma unroll
    for (int k = 0; k < F8_LAT_LOADS; ++k) issue_dma(d, k);
    if (rope_loader) issue_dma(d, F8_LAT_LOADS);
  };
  // this wave's loads of all tiles but the last one issued have landed (or of all of them)
  auto wait_ring = [&](bool keep_last) {
    if (!keep_last)
      wait_vmcnt<0>();
    else if (rope_loader)
      wait_vmcnt<F8_LAT_LOADS + 1>();
    else
      wait_vmcnt<F8_LAT_LOADS>();
  };
  issue(t_lo);
  if (t_lo + 1 < t_hi) issue(t_lo + 1);

  // ---- per-lane LDS read offsets
  // K row of this lane: the MFMA row order tau within the 32-token block, with the block's halves
  // swapped on dim half 1, so that accumulator elements 0..7 of lane (head, half h) are tokens
  // 16 dq + 8 h + 0..7 on both dim halves and elements 8..15 the tokens the other half keeps
  const int kr = 32 * tq + (tau(hh) ^ (16 * dq));
  const int fk = (2 * hf) ^ swz_lat(kr);   // latent chunk of k-step s: (4 s) ^ fk (+ 16 dq)
  const int fr = (2 * hf) ^ swz_rope(kr);  // rope chunks: fr, fr ^ 1
  // V^T operand of a 32-dim block: lane (dim l % 32, half h) holds tokens 16 h + 0..15 and
  // 32 + 16 h + 0..15, read as four 8-token transposes r = 0..3 at rows
  // 16 h + 8 (r & 1) + 32 (r >> 1) + (lane % 16) / 2; the swizzle depends on r & 1 only
  const int i16 = lane & 15, gq = lane >> 4;
  int vbase[2], vx[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int vrow = 16 * (gq >> 1) + 8 * par + (i16 >> 1);
    const int vu = (gq & 1) ^ swz_lat(vrow);
    vbase[par] = vrow * F8_DV + 16 * (vu & 1) + 8 * (i16 & 1);
    vx[par] = vu >> 1;
  }

  i32x8 qhi[4], qlo[4], qpe;
  int t = t_lo;
  int issued = t_lo + 1 < t_hi ? t_lo + 2 : t_lo + 1;  // tiles [t_lo, issued) requested
  int s_cur = 0;  // ring stage of tile t
  int cb = b_first;
  int cb_lo = ldc(a.cu + cb), cb_hi = ldc(a.cu + cb + 1);

  // Tile x becomes visible: this thread's loads of it have landed (only tile x + 1's may still
  // be in flight), then the workgroup barrier, after which every wave is also done with the
  // stage of tile x - 2. Returns whether tile x + 1 is to be loaded now (into that stage).
  auto visible = [&](int x, Dma& dma) {
    wait_ring(issued > x + 1);
    wg_barrier();
    if (issued == x + 1 && issued < t_hi) {
      dma = issue_setup(issued);
      ++issued;
      return true;
    }
    return false;
  };
  // Partial S^T of tile x for this wave's 32 tokens and dim half (rows past the sequence read as
  // zeros and are masked later), the LDS-DMA instructions of the refill spread over the first
  // k-steps (REFILL) and the work hook(i) after MFMA i (0..8). No branches inside.
  // Per-step waits: before k-step s, all but the LDS accesses issued by the hooks after the K read
  // of step s (W[s] of them) must have completed; the hooks of the softmax issue, after the K
  // read of step 1: 3 reads (hook 0); step 2: a write and, after a barrier, 1 read; step 4: a
  // write and, after a barrier, 2 reads.
  auto qk_body = [&](const uint8_t* st, f32x16& so, const Dma& dma, auto REFILLc, auto HOOKEDc,
                     auto&& hook) {
    constexpr bool REFILL = decltype(REFILLc)::value;
    constexpr bool HOOKED = decltype(HOOKEDc)::value;
    constexpr int W[5] = {0, HOOKED ? 3 : 0, HOOKED ? 1 : 0, 0, HOOKED ? 2 : 0};
    const uint8_t* krow = st + kr * F8_DV + 256 * dq;
    const uint8_t* prow = st + F8_LAT + kr * F8_DPE;
    i32x8 kop[2];
    auto kread = [&](int s) {  // s = 0..3 latent, 4 rope
      kop[s & 1] = s < 4 ? lds_2xb128(krow + 16 * ((4 * s) ^ fk), krow + 16 * (((4 * s) ^ fk) ^ 1))
                         : lds_2xb128(prow + 16 * fr, prow + 16 * (fr ^ 1));
    };
    kread(0);
    so = f32x16{};
#pragma unroll
    for (int s = 0; s < 5; ++s) {
      lgkm_wait(W[s]);  // the K read of k-step s has completed
      order_after(kop[s & 1]);
      if (s + 1 < 5) kread(s + 1);
      if constexpr (REFILL) {
        if (s < F8_LAT_LOADS / 2) {
          issue_dma(dma, 2 * s);
          issue_dma(dma, 2 * s + 1);
        }
        if (s == F8_LAT_LOADS / 2 && rope_loader) issue_dma(dma, F8_LAT_LOADS);
      }
      if (s < 4) {
        so = mfma_fp8(kop[s & 1], qhi[s], so);
        hook(2 * s);
        so = mfma_fp8(kop[s & 1], qlo[s], so);
        hook(2 * s + 1);
      } else {
        so = mfma_fp8(kop[s & 1], qpe, so);
        hook(8);
      }
      sched_fence();
    }
  };
  auto qk = [&](const uint8_t* st, f32x16& so, bool refill, const Dma& dma, auto HOOKEDc,
                auto&& hook) {
    if (refill)
      qk_body(st, so, dma, std::true_type{}, HOOKEDc, hook);
    else
      qk_body(st, so, dma, std::false_type{}, HOOKEDc, hook);
  };

  while (t < t_hi) {  // one iteration per sequence piece
    while (t >= cb_hi) {
      ++cb;
      cb_lo = cb_hi;
      cb_hi = ldc(a.cu + cb + 1);
    }
    const int L = max(0, min(ldc(a.seqlens + cb), a.lmax));
    const int64_t qr = (int64_t)cb * a.Hq + head;
    const float ch = a.score_scale * kvs * load_q(a, qr, dq, hf, qhi, qlo, qpe);
    const int p_lo = t, p_hi = min(t_hi, cb_hi);
    const bool complete = p_lo == cb_lo && p_hi == cb_hi;
    const int slot = p_lo == t_lo ? 0 : 1;
    bool have_scr = false, first = true;
    float lse_scr = 0.f, mref = 0.f, lsum = 0.f;
    f32x16 oacc[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) oacc[d] = f32x16{};
    const int dbase = 128 * q + 4 * hf;  // first output dim of this lane

    // Segment end: normalise, merge with an earlier segment (scratch slot), store this wave's
    // 128 dims: to the output for a complete sequence, else to the piece's partial slot (a cut
    // segment goes to the scratch slot). Partial slots are [slot][head][512] bf16.
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
      auto slot_row = [&](int64_t sb) {
        return (u32x2*)(a.part_o + (sb * a.Hq + head) * F8_DV + dbase);
      };
      const u32x2* scr = slot_row((int64_t)g * F8_SLOTS + 2);
      // value of output group (dt, q4) of this lane: dims 32 dt + 8 q4 + 0..3 past dbase
      auto val = [&](int dt, int q4, auto merge) {
        f32x4 v = {oacc[dt][4 * q4], oacc[dt][4 * q4 + 1], oacc[dt][4 * q4 + 2],
                   oacc[dt][4 * q4 + 3]};
        v *= w_seg;
        if constexpr (decltype(merge)::value) v += bf16x4_to_f32(scr[8 * dt + 2 * q4]) * w_old;
        return v;
      };
      auto store = [&](auto merge) {
        if (cut || !complete) {
          const int64_t sb = (int64_t)g * F8_SLOTS + (cut ? 2 : slot);
          u32x2* dst = slot_row(sb);
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              const f32x4 v = val(dt, q4, merge);
              dst[8 * dt + 2 * q4] =
                  u32x2{h16<true>::pack(v[0], v[1]), h16<true>::pack(v[2], v[3])};
            }
            sched_fence();
          }
          if (q == 0 && hf == 0) a.part_lse[sb * a.Hq + head] = lse_out;
        } else {
          using H = h16<O_BF16>;
          uint16_t* o = a.out + qr * F8_DV + dbase;
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
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
      wait_vmcnt<0>();  // stores retire before the ring's vmcnt accounting resumes
      if (cut) {
        have_scr = true;
        lse_scr = lse_out;
      }
    };

    // partial scores: elements 8..15 go to the other dim half, 0..7 are kept (raw, unmasked)
    float s8[8];
    auto publish = [&](const f32x16& sv) {
      xs[hb][tq][dq ^ 1][0][lane] = f32x4{sv[8], sv[9], sv[10], sv[11]};
      xs[hb][tq][dq ^ 1][1][lane] = f32x4{sv[12], sv[13], sv[14], sv[15]};
#pragma unroll
      for (int i = 0; i < 8; ++i) s8[i] = sv[i];
    };

    // prologue: partial S^T of the piece's first tile
    {
      Dma dma{};
      const bool refill = visible(t, dma);
      f32x16 s0;
      qk(stage(s_cur), s0, refill, dma, std::false_type{}, [](int) {});
      publish(s0);
    }
    for (; t < p_hi; ++t, s_cur = next_stage(s_cur)) {
      const uint8_t* st = stage(s_cur);
      // valid tokens of this wave's 16 (kept element i of lane half h is token 8 h + i of them)
      const int own = L - (t - cb_lo) * F8_TILE - 32 * tq - 16 * dq;
      const bool nxt = t + 1 < p_hi;
      // Softmax of tile t as short levels of independent instructions, one after each MFMA of
      // the next tile's S^T (the wave issues in order, so a dependent chain between two MFMAs
      // would hold back the second). LDS accesses are inline asm with explicit waits.
      //   0: other half's partial scores, and the previous tile's row sums
      //   1: add, mask, 8-element max; previous tile's row sum into lsum
      //   2: lane-half max -> LDS (16-token maxima)
      //   3: barrier B, read the head block's four maxima
      //   4: tile max, segment check, block scales
      //   5: exponentials
      //   6: P^T in e4m3 -> LDS, rounded P back to float
      //   7: barrier C, read the B operand (both token blocks); pairwise sums
      //   8: 16-token sum of the rounded P -> LDS (read with the next tile)
      float sh = 0.f, m_old = 0.f, mb = 0.f;
      int es_me = 0, psc = 0;
      bool cut = false;  // a new segment starts at this tile (flushed before its O^T update)
      int phi[2];
      float pr[8], a4[4];
      i32x8 pbh;
      i32x4 xin0, xin1, x4, m4;
      auto hook = [&](int k, auto HOOKEDc) {
        constexpr bool HOOKED = decltype(HOOKEDc)::value;
        if (k == 0) {
          xin0 = lds_b128(&xs[hb][tq][dq][0][lane]);
          xin1 = lds_b128(&xs[hb][tq][dq][1][lane]);
          x4 = lds_b128(&xsum[hb][hh]);
        }
        if (k == 1) {
          lgkm<0>();
          order_after(xin0);
          order_after(xin1);
          order_after(x4);
          const f32x4 p0 = as_f32x4(xin0), p1 = as_f32x4(xin1), pv = as_f32x4(x4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s8[e] += p0[e];
            s8[4 + e] += p1[e];
          }
          if (own < 16) {  // wave-uniform: the sequence ends inside this wave's tokens
#pragma unroll
            for (int i = 0; i < 8; ++i) s8[i] = 8 * hf + i >= own ? -INFINITY : s8[i];
          }
          mb = fmaxf(fmaxf(fmaxf(s8[0], s8[1]), fmaxf(s8[2], s8[3])),
                     fmaxf(fmaxf(s8[4], s8[5]), fmaxf(s8[6], s8[7])));
          // the previous tile's sum (same order on the four waves), unless this tile starts
          // the piece
          if (t > p_lo) lsum += (pv[0] + pv[1]) + (pv[2] + pv[3]);
        }
        if (k == 2) {
          // raw scores; the log2-domain scale ch > 0 is applied inside exp2
          mb = xhalf_max(mb) * ch;
          lds_write_b32((float*)&xmax[hb][hh] + q, __float_as_uint(mb));
        }
        if (k == 3) {
          wg_barrier();
          m4 = lds_b128(&xmax[hb][hh]);
        }
        if (k == 4) {
          if constexpr (HOOKED)
            lgkm<2>();  // the K read issued after it may still be in flight
          else
            lgkm<0>();
          order_after(m4);
          const f32x4 mx = as_f32x4(m4);
          const float mt = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));  // tile max
          // a tile whose max exceeds the reference by more than the headroom ends the segment;
          // P of this tile then uses the new reference and the old segment is flushed after the
          // S^T MFMAs (wave-uniform decision, the same on the head block's four waves)
          cut = !first && __ballot(mt > mref + F8_RESET) != 0;
          m_old = mref;
          mref = (first || cut) ? mt : mref;
          first = false;
          // P^T of a 32-token block in e4m3 on a per-head power-of-two scale 2^es, es =
          // floor(block max - reference) - 7, so the block's largest scaled P lies in [128, 256);
          // folded into the exp2 argument and passed to the O^T MFMA as the block's E8M0 scale.
          // The row sums add the rounded P, so the weights applied to V sum to one and the
          // largest P of a segment, 2^0, is exact
          auto bscale = [&](float mblk) {
            const int e = (int)floorf(mblk - mref) - 7;
            return mblk == -INFINITY ? 0 : max(-127, min(127, e));
          };
          const int es0 = bscale(fmaxf(mx[0], mx[2])), es1 = bscale(fmaxf(mx[1], mx[3]));
          es_me = tq ? es1 : es0;
          psc = (hf ? es1 : es0) + 127;  // the scale of k block h comes from lane half h
          sh = -(mref + (float)es_me);
        }
        if (k == 5) {
#pragma unroll
          for (int i = 0; i < 8; ++i) pr[i] = fmaf(s8[i], ch, sh);
#pragma unroll
          for (int i = 0; i < 8; ++i) pr[i] = __builtin_amdgcn_exp2f(pr[i]);
        }
        if (k == 6) {
          phi[0] = pack_fp8x4(pr[0], pr[1], pr[2], pr[3]);
          phi[1] = pack_fp8x4(pr[4], pr[5], pr[6], pr[7]);
          lds_write_b64(&xq[hb][tq][dq][hh][8 * hf], u32x2{(uint32_t)phi[0], (uint32_t)phi[1]});
          typedef float f2 __attribute__((ext_vector_type(2)));
#pragma unroll
          for (int w = 0; w < 2; ++w) {
            const f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(phi[w], false);
            const f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(phi[w], true);
            pr[4 * w] = lo[0];
            pr[4 * w + 1] = lo[1];
            pr[4 * w + 2] = hi[0];
            pr[4 * w + 3] = hi[1];
          }
        }
        if (k == 7) {
          wg_barrier();
          // B operand: lane (head hh, half h) holds tokens 16 h + 0..15 of both token blocks
          pbh = lds_2xb128(&xq[hb][0][hf][hh][0], &xq[hb][1][hf][hh][0]);
#pragma unroll
          for (int i = 0; i < 4; ++i) a4[i] = pr[2 * i] + pr[2 * i + 1];
        }
        if (k == 8) {
          const float ps = xhalf_sum(ldexpf((a4[0] + a4[1]) + (a4[2] + a4[3]), es_me));
          lds_write_b32((float*)&xsum[hb][hh] + q, __float_as_uint(ps));
        }
      };
      f32x16 sn;
      if (nxt) {
        Dma dma{};
        const bool refill = visible(t + 1, dma);
        qk(stage(next_stage(s_cur)), sn, refill, dma, std::true_type{},
           [&](int k) { hook(k, std::true_type{}); });
      } else {
        wg_barrier();  // the partial scores of tile t are published
#pragma unroll
        for (int k = 0; k < 9; ++k) hook(k, std::false_type{});
      }
      if (cut) {  // wave-uniform; rare
        flush(true, m_old);
#pragma unroll
        for (int d = 0; d < 4; ++d) oacc[d] = f32x16{};
        lsum = 0.f;
      }
      // O^T (this wave's 128 dims) += V^T P^T over the tile's 64 tokens: 4 dim blocks
      auto vread = [&](int dt) {
        i32x2 r[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          r[rr] = lds_tr8(st + vbase[rr & 1] + 32 * F8_DV * (rr >> 1) +
                          32 * ((4 * q + dt) ^ vx[rr & 1]));
        return i32x8{r[0][0], r[0][1], r[1][0], r[1][1], r[2][0], r[2][1], r[3][0], r[3][1]};
      };
      i32x8 vop[2];
      vop[0] = vread(0);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        if (dt + 1 < 4) {
          vop[(dt + 1) & 1] = vread(dt + 1);
          lgkm_wait(4);  // all but the 4 reads just issued
        } else {
          lgkm_wait(0);
        }
        order_after(vop[dt & 1]);
        if (dt == 0) order_after(pbh);
        oacc[dt] = mfma_fp8_bscaled(vop[dt & 1], pbh, oacc[dt], psc);
        sched_fence();
      }
      if (nxt) publish(sn);
    }
    // the last tile's row sums
    wg_barrier();
    {
      const f32x4 pv = xsum[hb][hh];
      lsum += (pv[0] + pv[1]) + (pv[2] + pv[3]);
    }
    flush(false, mref);
  }
}

// ------------------------------------------------------------------------------------------------
// 128 heads per workgroup (Hq a multiple of 128): 4 waves, one per SIMD, each owning 32 heads for
// the whole tile: S^T = K Q^T, the softmax and O^T = V^T P^T with no exchange between waves, so
// the only barrier per tile hands over the ring, and each KV tile goes from L2 to LDS once for all
// 128 heads.
//   * registers: the 32 heads' O^T (512 dims: 256 fp32 accumulators per lane, all the AGPRs)
//     and the hi term of Q (72 VGPRs); S^T accumulates in VGPRs (inline-asm MFMA, since the
//     builtin's AGPR form would take AGPRs from O^T); the lo term of Q is kept in LDS (one wave's
//     32 heads: 18 KB) and read with K;
//   * a 64-token tile is two 32-token blocks b; K rows are fed to the S^T MFMA in the order rho
//     (row m -> token (m & 3) | ((m >> 3) & 3) << 2 | ((m >> 2) & 1) << 4), so accumulator element
//     i of lane half h is token 16 h + i of the block: packed to e4m3 they are exactly bytes
//     16 b .. 16 b + 15 of the P^T operand of lane half h, with no exchange between lanes;
//   * the S^T MFMAs of both blocks are one stream of 18 k-steps with LDS reads two k-steps ahead;
//     block 0's softmax runs between block 1's MFMAs, block 1's after them; the row sums of the
//     rounded, scaled P come from one more MFMA (ones^T P^T) with the O^T update;
//   * references are whole numbers, so moving one (a block more than 64 above it) scales the
//     accumulated O^T and row sums by an exact power of two, in place in the AGPRs (rare);
//   * 2-stage ring: the tile is consumed (S^T then O^T) within one iteration, and the next tile
//     is loaded meanwhile (9 LDS-DMA instructions per wave, on the even k-steps of the stream);
//   * the ring's 16-byte chunks are swizzled with row bits 0..2 and 4 (the rows read together
//     under the order rho differ there), which keeps the K row reads, the rope reads and the
//     transposed V reads free of bank conflicts;
//   * at a piece end the next piece's Q is requested first, then the normalised rows are staged
//     through the last tile's ring stage and stored whole; the next piece's first tile waits for
//     the loads only (the stores are the most recent VMEM operations).
constexpr int W_HEADS = 128;
constexpr int W_NSTAGE = 2;
constexpr int W_QLO = 9 * 64 * 32;  // one wave's Q lo operands: [k-step][16-byte half][lane]

TLM_DEV int w_rho(int m) { return (m & 3) | (((m >> 3) & 3) << 2) | (((m >> 2) & 1) << 4); }
TLM_DEV int w_swz(int r) { return ((r & 7) << 1) | ((r >> 4) & 1); }
TLM_DEV int w_swz_rope(int r) { return (((r >> 2) & 1) << 1) | ((r >> 4) & 1); }

template <bool O_BF16>
__global__ __launch_bounds__(256, 1) void mla_fp8_decode_w32(const F8Args a) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[W_NSTAGE * F8_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t qlo_lds[4][W_QLO];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) index
  const int hh = lane & 31, hf = lane >> 5;
  const int HG = a.Hq / W_HEADS;
  const F8Work wk = f8_work(blockIdx.x, HG);
  if (wk.g >= a.G) return;
  const int g = wk.g, hgi = wk.hgi;
  const int head0 = hgi * W_HEADS + 32 * wave;  // the wave's first head (uniform)
  const int head = head0 + hh;
  // tile indices fit int32 (the tile prefix is int32)
  const int t_lo = ldc(a.range_t + g), t_hi = ldc(a.range_t + g + 1);
  if (t_lo >= t_hi) return;
  const float kvs = a.kv_scale ? ldc(a.kv_scale) : 1.0f;

  // ---- per-tile page table: lane j holds the first KV row of tile tb + j and the number of its
  // rows to load (the sequence's valid tokens that lie inside the pool; the rest read as zeros)
  int tb = INT32_MIN / 2;
  uint32_t tab_lo = 0, tab_hi = 0;
  int tab_n = 0, tab_b = 0;
  auto build_table = [&](int base) {
    tb = base;
    const int tj = base + lane;
    tab_lo = tab_hi = 0;
    tab_n = 0;
    if (tj < t_hi) {
      int blo = 0, bhi = a.B - 1;  // largest b with cu[b] <= tj
      while (blo < bhi) {
        const int mid = (blo + bhi + 1) >> 1;
        if (a.cu[mid] <= tj) blo = mid; else bhi = mid - 1;
      }
      tab_b = blo;
      const F8Seg sg = f8_seg(a, blo, a.seqlens[f8_seq(a, blo)]);
      const int tok0 = (tj - a.cu[blo]) * F8_TILE;  // within the segment
      const int valid = min(F8_TILE, sg.len - tok0);
      const int tk = sg.start + tok0;  // within the sequence
      const int64_t row0 =
          (int64_t)a.bt[(int64_t)sg.b * a.max_pages + tk / a.page] * a.page + tk % a.page;
      int64_t nrow = min((int64_t)valid, a.kv_rows - row0);
      if (row0 < 0 || nrow < 0) nrow = 0;
      tab_lo = (uint32_t)row0;
      tab_hi = (uint32_t)((uint64_t)row0 >> 32);
      tab_n = (int)nrow;
    }
  };
  build_table(t_lo);
  // first sequence with a tile in [t_lo, t_hi): the sequence of lane 0's tile
  const int b_first = __builtin_amdgcn_readfirstlane(tab_b);

  // ---- KV ring: LDS-DMA of tile t into stage (t - t_lo) % 2; wave w loads latent rows
  // 16 w .. 16 w + 15 (8 instructions) and rope rows 16 w .. 16 w + 15 (1 instruction)
  struct Dma {  // one tile's source rows (base, byte count) and ring stage
    const uint8_t* bkv;
    const uint8_t* bpe;
    int nkv, npe;
    uint8_t* st;
  };
  auto stage = [&](int si) { return ring + si * F8_STAGE; };
  int s_issue = 0;  // ring stage of the next tile to request
  auto issue_setup = [&](int t) {
    if (t >= tb + 64) build_table(t);
    const int j = t - tb;
    const int64_t row0 = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)tab_hi, j) << 32) |
                                   (uint32_t)__builtin_amdgcn_readlane((int)tab_lo, j));
    const int64_t nrow = __builtin_amdgcn_readlane(tab_n, j);
    const uint8_t* bkv = nrow > 0 ? a.kv + row0 * a.kv_stride : a.kv;
    const uint8_t* bpe = nrow > 0 ? a.k_pe + row0 * a.kpe_stride : a.k_pe;
    const Dma d{bkv, bpe, (int)(nrow * a.kv_stride), (int)(nrow * a.kpe_stride), stage(s_issue)};
    s_issue ^= 1;
    return d;
  };
  // latent instruction k (0..7) of lane (c, h) = (lane % 32, lane / 32) reads row r = 16 w + 2 k + h
  // at swizzled chunk c ^ w_swz(r) = (c ^ (2 h + (w & 1))) ^ 4 (k % 4)
  const int lat_off = (16 * wave + hf) * (int)a.kv_stride;
  const int lat_x16 = 16 * (hh ^ (2 * hf + (wave & 1)));
  auto issue_dma = [&](const Dma& d, int k) {
    if (k < 8) {  // latent: 2 rows x 32 chunks per wave-instruction
      int lo = lat_off, lx = lat_x16;
      asm volatile("" : "+v"(lo), "+v"(lx));  // per use: the 9 offsets are not kept live
      const int off = lo + 2 * k * (int)a.kv_stride + (lx ^ (64 * (k & 3)));
      const __amdgpu_buffer_rsrc_t rk =
          __builtin_amdgcn_make_buffer_rsrc((void*)d.bkv, (short)0, d.nkv, F8_RSRC_WORD3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(d.st + (8 * wave + k) * 1024), 16,
                                               off, 0, 0, F8_KV_NT);
    } else {  // rope: 16 rows x 4 chunks per wave-instruction
      int ln;  // lane id computed here, not kept in a register across the tile
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
      const int r = 16 * wave + (ln >> 2);
      const int off = r * (int)a.kpe_stride + 16 * ((ln & 3) ^ w_swz_rope(r));
      const __amdgpu_buffer_rsrc_t rp =
          __builtin_amdgcn_make_buffer_rsrc((void*)d.bpe, (short)0, d.npe, F8_RSRC_WORD3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, (lds_void*)(d.st + F8_LAT + wave * 1024), 16,
                                               off, 0, 0, F8_KV_NT);
    }
  };
  {
    const Dma d = issue_setup(t_lo);
#pragma unroll
    for (int k = 0; k < 9; ++k) issue_dma(d, k);
  }

  // ---- per-lane LDS read offsets within a ring stage (stages are 1024-byte aligned, so adding a
  // stage base leaves bits 4..9 of an offset as they are and a swizzle step is one XOR there).
  // K row of this lane in block b: 32 b + rho(lane % 32); its latent 32-byte chunk of k-step s
  // is (kofs[b] ^ 64 s) and (kofs[b] ^ 64 s ^ 16), its rope chunk at pofs[b]
  const int kr0 = w_rho(hh);
  int kofs[2], pofs[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int r = 32 * b + kr0;
    kofs[b] = r * F8_DV + 16 * ((2 * hf) ^ w_swz(r));
    pofs[b] = F8_LAT + r * F8_DPE + 16 * ((2 * hf) ^ w_swz_rope(r));
  }
  // V^T operand of a 32-dim block dt: lane (dim l % 32, half h) holds tokens 16 h + 0..15 and
  // 32 + 16 h + 0..15, read as four 8-token transposes r = 0..3 at rows
  // 16 h + 8 (r & 1) + 32 (r >> 1) + (lane % 16) / 2, i.e. at (vofs[r & 1] ^ 32 dt) and 32 rows
  // (16 KB) further; the swizzle depends on r & 1 only
  const int i16 = lane & 15, gq = lane >> 4;
  int vofs[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int vrow = 16 * (gq >> 1) + 8 * par + (i16 >> 1);
    const int vu = (gq & 1) ^ w_swz(vrow);
    vofs[par] = vrow * F8_DV + 16 * (vu & 1) + 8 * (i16 & 1) + 32 * (vu >> 1);
  }
  uint8_t* const qlo_w = qlo_lds[wave];
  // Q lo of k-step s: bytes 0..15 of every lane, then bytes 16..31 (1 KB each, read whole)
  const uint32_t qlo_a = lds_addr(qlo_w) + 16 * lane;

  i32x8 qhi[9];
  int t = t_lo;
  int s_cur = 0;  // ring stage of tile t
  int cb = b_first;
  int cb_lo = ldc(a.cu + cb), cb_hi = ldc(a.cu + cb + 1);

  // S^T of both 32-token blocks of the tile in stage st as one stream of 18 k-steps (rows past
  // the sequence read as zeros and are masked later): k-step j is k-step j % 9 of block j / 9.
  // LDS reads run KD k-steps ahead across the block boundary; the last KD k-steps issue the
  // first KD V^T reads of the O^T update instead (vpre). The even k-steps carry the LDS-DMA
  // instructions of a refill (DMA); block 1's MFMAs carry the work hook(i) after MFMA i
  // (0..17). No branches inside: the k-steps form one block.
  constexpr int KD = 2;
  auto qk_body = [&](const uint8_t* st, f32x16& s0, f32x16& s1, const Dma& dma, auto DMAc,
                     auto&& hook, auto&& vpre) {
    constexpr bool DMA = decltype(DMAc)::value;
    const uint32_t sa = lds_addr(st);
    i32x8 kop[KD + 1], qop[KD + 1];
    auto kread = [&](auto Jc) {  // K bytes and this lane's Q lo bytes of k-step j
      constexpr int j = decltype(Jc)::value, b = j / 9, s = j % 9;
      const uint32_t a0 = s < 8 ? (sa + kofs[b]) ^ (64 * s) : sa + pofs[b], a1 = a0 ^ 16;
      const i32x4 k0 = lds_b128_off<0>(a0), k1 = lds_b128_off<0>(a1);
      const i32x4 q0 = lds_b128_off<s * 64 * 32>(qlo_a);
      const i32x4 q1 = lds_b128_off<s * 64 * 32 + 64 * 16>(qlo_a);
      kop[j % (KD + 1)] = i32x8{k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
      qop[j % (KD + 1)] = i32x8{q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
    };
    static_for<KD>([&](auto Jc) { kread(Jc); });
    static_for<18>([&](auto Jc) {
      constexpr int j = decltype(Jc)::value, b = j / 9, s = j % 9, u = j % (KD + 1);
      f32x16& so = b ? s1 : s0;
      // the 4 reads of k-step j have completed; the KD - 1 later batches of 4 may be
      // outstanding (every k-step issues one batch; the hooks issue no LDS accesses)
      lgkm<4 * (KD - 1)>();
      order_after(kop[u]);
      order_after(qop[u]);
      if constexpr (j + KD < 18)
        kread(std::integral_constant<int, j + KD>{});
      else
        vpre(j + KD - 18);
      // the refill, spread over both blocks (even k-steps): the CU takes each 1 KB LDS-DMA
      // instruction in ~40 cycles, which a burst on block 0 alone turned into issue stalls
      if constexpr (DMA && j % 2 == 0) issue_dma(dma, j / 2);
      if constexpr (s == 0)
        mfma_fp8_v0(so, kop[u], qhi[0]);
      else
        mfma_fp8_v(so, kop[u], qhi[s]);
      if constexpr (b == 1) hook(2 * s);
      mfma_fp8_v(so, kop[u], qop[u]);
      if constexpr (b == 1) hook(2 * s + 1);
      if constexpr (j == 8) xdl_settle();  // before block 1's hooks read s0
      sched_fence();
    });
    xdl_settle();  // before the softmax reads s1
  };
  auto qk = [&](const uint8_t* st, f32x16& s0, f32x16& s1, bool dma_on, const Dma& dma,
                auto&& hook, auto&& vpre) {
    if (dma_on)
      qk_body(st, s0, s1, dma, std::true_type{}, hook, vpre);
    else
      qk_body(st, s0, s1, dma, std::false_type{}, hook, vpre);
  };

  // Q of the piece starting at tile t: its sequence cb, the hi term into VGPRs, the lo term
  // straight into this wave's LDS area (LDS-DMA, 18 x 1 KB: lane l's 16 bytes land at l * 16)
  // and the exponent (asm load: waited for with the rest at the piece's first tile)
  int L = 0, qe = 0;
  auto begin_piece = [&]() {
    while (t >= cb_hi) {
      ++cb;
      cb_lo = cb_hi;
      cb_hi = ldc(a.cu + cb + 1);
    }
    const F8Seg sg = f8_seg(a, cb, ldc(a.seqlens + f8_seq(a, cb)));
    L = sg.len;
    const int64_t qr0 = (int64_t)sg.b * a.Hq + head0;  // the wave's first Q row (uniform)
    const uint8_t* qs = a.qsplit + (qr0 + hh) * F8_QROW;
#pragma unroll
    for (int s = 0; s < 9; ++s) qhi[s] = *(const i32x8*)(qs + 64 * s + 32 * hf);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.qsplit + qr0 * F8_QROW), (short)0, 32 * F8_QROW, F8_RSRC_WORD3);
    int ln;  // lane id computed here: a lane offset hoisted out of the piece loop is spilled
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    const int qoff = (ln & 31) * F8_QROW + F8_DV + F8_DPE + 32 * (ln >> 5);
    static_for<18>([&](auto Ic) {  // k-step i / 2, 16-byte half i % 2
      // the step goes in soffset: an instruction offset would also move the LDS destination
      constexpr int i = decltype(Ic)::value;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void*)(qlo_w + i * 1024), 16, qoff,
                                               64 * (i / 2) + 16 * (i % 2), 0, 0);
    });
    asm volatile("global_load_dword %0, %1, off" : "=v"(qe) : "v"(a.qexp + qr0 + hh) : "memory");
  };
  begin_piece();

  // Piece end: the wave's 32 heads x 512 dims, normalised, go to the output for a complete
  // sequence, else to the piece's partial slot ([slot][head][512] bf16) with its lse. Rows go
  // out whole: each quarter (128 dims) is staged in this wave's quarter of the ring stage the
  // piece's last tile used (all waves are past it: barrier), as [head][128] with 16-byte chunk c
  // of head h at c ^ (h % 16), and read back as four 256-byte head rows per instruction. The
  // lse store comes first, then exactly FLUSH_STORES row stores.
  constexpr int FLUSH_STORES = 32;
  auto flush = [&](f32x16 (&oacc)[16], uint16_t* rows, float* lse_at, float lse, float w,
                   const uint8_t* stg, auto H) {
    using HH = decltype(H);
    // lane terms computed here from an opaque lane id: hoisted out of the piece loop they
    // would be kept in (spilled) registers across it
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    const int lh = ln & 31, lf = ln >> 5, l16 = ln & 15, l4 = ln >> 4;
    if (lse_at && lf == 0) *lse_at = lse;
    const uint32_t stage_a = lds_addr(stg) + wave * (F8_STAGE / 4);
    // the wave's 32 rows as one buffer (base wave-uniform, offsets 32-bit)
    const __amdgpu_buffer_rsrc_t orows =
        __builtin_amdgcn_make_buffer_rsrc((void*)rows, (short)0, 32 * F8_DV * 2, F8_RSRC_WORD3);
#pragma unroll
    for (int h4 = 0; h4 < 4; ++h4) {
#pragma unroll
      for (int d4 = 0; d4 < 4; ++d4) {
        const int dt = 4 * h4 + d4;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {  // dims 32 dt + 8 q4 + 4 hf + 0..3 of head hh
          const f32x4 v = f32x4{oacc[dt][4 * q4], oacc[dt][4 * q4 + 1], oacc[dt][4 * q4 + 2],
                                oacc[dt][4 * q4 + 3]} * w;
          lds_write_b64_at(stage_a + lh * 256 + 16 * ((4 * d4 + q4) ^ (lh & 15)) + 8 * lf,
                           u32x2{HH::pack(v[0], v[1]), HH::pack(v[2], v[3])});
        }
        oacc[dt] = f32x16{};  // ready for the next piece (before the stores below are issued)
        sched_fence();
      }
      lgkm<0>();
      i32x4 x[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {  // heads 4 i + l4, chunk l16
        const int hr = 4 * i + l4;
        x[i] = lds_b128_off<0>(stage_a + hr * 256 + 16 * (l16 ^ (hr & 15)));
      }
      lgkm<0>();
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        order_after(x[i]);
        const int hr = 4 * i + l4;
        __builtin_amdgcn_raw_buffer_store_b128(x[i], orows, hr * 2 * F8_DV + 256 * h4 + 16 * l16,
                                               0, F8_ROW_CP);
      }
    }
  };

  f32x16 oacc[16];  // O^T of the piece; zero at its start (the flush clears it)
#pragma unroll
  for (int d = 0; d < 16; ++d) oacc[d] = f32x16{};
  while (t < t_hi) {  // one iteration per sequence piece
    const int p_lo = t, p_hi = min(t_hi, cb_hi);
    const bool complete = p_lo == cb_lo && p_hi == cb_hi;
    const int slot = p_lo == t_lo ? 0 : 1;
    const float ch = a.score_scale * kvs;  // times 2^qe, applied at the piece's first tile
    float chq = 0.f;
    bool first = true;
    float mref = 0.f, lsum = 0.f;

    // References are whole numbers (log2 domain), so a change of reference is a power of two:
    // a block whose max exceeds the reference by more than the headroom moves it to the block
    // max rounded up, and what was accumulated under the old one is scaled by 2^(old - new)
    // (rare, wave-uniform)
    while (t < p_hi) {
      // tile t visible: this wave's loads of it have landed, then every wave's (barrier), after
      // which the other stage (tile t - 1) is free for tile t + 1. At a piece's first tile the
      // previous piece's row stores (the most recent VMEM operations) may still be in flight;
      // the piece's Q was requested before them.
      if (t == p_lo && p_lo != t_lo) {
        wait_vmcnt<FLUSH_STORES>();
      } else {
        wait_vmcnt<0>();
      }
      wg_barrier();
      if (t == p_lo) {
        asm volatile("" : "+v"(qe) : : "memory");  // the exponent is read after the wait
        chq = ch * ldexpf(1.0f, qe);
      }
      Dma dma{};
      const bool refill = t + 1 < t_hi;
      if (refill) dma = issue_setup(t + 1);
      const uint8_t* st = stage(s_cur);
      // valid tokens of the tile's two 32-token blocks (element i of lane half h is token
      // 16 h + i of its block)
      const int own0 = L - (t - cb_lo) * F8_TILE, own1 = own0 - 32;

      // softmax of one 32-token block, as levels placed after the MFMAs of the next S^T block
      // (or run back to back): mask and 8-of-16 max; lane-half max and segment check; block
      // scale; exponentials; e4m3 pack; rounded sums
      struct Blk {
        float mb, sh;
        int es;
        bool cut;
        float m_old;
        float p[16];
        int w[4];
      };
      auto smax = [&](f32x16& sv, int own, Blk& k, int lvl) {
        if (lvl == 0) {
          if (own < 32) {  // wave-uniform: the sequence ends inside this block (a branch, not
                           // selects on every tile)
            asm volatile("" ::: "memory");
#pragma unroll
            for (int i = 0; i < 16; ++i) sv[i] = 16 * hf + i >= own ? -INFINITY : sv[i];
          }
          float m8[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            m8[j] = fmaxf(fmaxf(sv[4 * j], sv[4 * j + 1]), fmaxf(sv[4 * j + 2], sv[4 * j + 3]));
          k.mb = fmaxf(fmaxf(m8[0], m8[1]), fmaxf(m8[2], m8[3]));
        }
        if (lvl == 1) {
          // raw scores; the log2-domain scale ch > 0 is applied inside exp2. A head whose block
          // max exceeds its reference by more than the headroom moves the reference up to the
          // block max rounded up; the rescale runs when any head of the wave moved (k.cut)
          k.mb = xhalf_max(k.mb) * chq;
          const bool over = first || k.mb > mref + F8_RESET;
          k.cut = !first && __ballot(over) != 0;
          k.m_old = mref;
          mref = over ? ceilf(k.mb) : mref;
          first = false;
        }
        if (lvl == 2) {
          // P^T in e4m3 on a per-head power-of-two scale 2^es, es = floor(block max - reference)
          // - 7, so the block's largest scaled P lies in [128, 256): folded into the exp2
          // argument and passed to the O^T MFMA as the block's E8M0 scale. The row sums add the
          // rounded P, so the weights applied to V sum to one
          const int e = (int)floorf(k.mb - mref) - 7;
          k.es = k.mb == -INFINITY ? 0 : max(-127, min(127, e));
          k.sh = -(mref + (float)k.es);
        }
        if (lvl >= 3 && lvl <= 10) {  // exponentials, two per level
          const int e = 2 * (lvl - 3);
          k.p[e] = __builtin_amdgcn_exp2f(fmaf(sv[e], chq, k.sh));
          k.p[e + 1] = __builtin_amdgcn_exp2f(fmaf(sv[e + 1], chq, k.sh));
        }
        if (lvl == 11 || lvl == 12) {
          const int q = 2 * (lvl - 11);
          k.w[q] = pack_fp8x4(k.p[4 * q], k.p[4 * q + 1], k.p[4 * q + 2], k.p[4 * q + 3]);
          k.w[q + 1] = pack_fp8x4(k.p[4 * q + 4], k.p[4 * q + 5], k.p[4 * q + 6], k.p[4 * q + 7]);
        }
      };
      // the row sums of the rounded, scaled P come from an MFMA; level i of block 0 runs after
      // block 1's MFMA LVL_AT[i] (dependent levels an MFMA apart at least)
      constexpr int NLVL = 13;
      constexpr int LVL_AT[NLVL] = {0, 2, 4, 5, 6, 7, 8, 9, 10, 11, 12, 14, 16};

      // V^T operand of 32-dim block dt; the reads run VD dim blocks ahead of the O^T MFMAs, the
      // first VD issued by the last k-steps of the S^T stream
      constexpr int VD = KD;
      const uint32_t va0 = lds_addr(st) + vofs[0], va1 = lds_addr(st) + vofs[1];
      i32x8 vop[VD + 1];
      auto vread = [&](int dt) {
        const uint32_t p0 = va0 ^ (32 * dt), p1 = va1 ^ (32 * dt);
        const i32x2 r0 = lds_tr8_off<0>(p0), r1 = lds_tr8_off<0>(p1);
        const i32x2 r2 = lds_tr8_off<32 * F8_DV>(p0), r3 = lds_tr8_off<32 * F8_DV>(p1);
        vop[dt % (VD + 1)] = i32x8{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
      };

      f32x16 s0, s1;
      Blk k0, k1;
      // S^T of both blocks (with the refill of tile t + 1 in block 0), block 0's softmax between
      // block 1's MFMAs, then block 1's through its e4m3 words
      qk(st, s0, s1, refill, dma, [&](int i) {
#pragma unroll
        for (int l = 0; l < NLVL; ++l)
          if (LVL_AT[l] == i) smax(s0, own0, k0, l);
      }, vread);
#pragma unroll
      for (int i = 0; i < NLVL; ++i) smax(s1, own1, k1, i);
      // O^T (512 dims) += V^T P^T over the tile's 64 tokens: 16 dim blocks, the rounded-sum
      // levels of block 1 placed between them
      // and, after the first dim block, the row sums of the tile's scaled P: ones^T P^T (every
      // output row holds them; the first MFMA has read P^T, so no VALU write precedes it)
      const i32x8 ones = i32x8{0x38383838, 0x38383838, 0x38383838, 0x38383838,
                               0x38383838, 0x38383838, 0x38383838, 0x38383838};  // e4m3 1.0
      auto pv = [&](const i32x8& pb, int psc) {
        f32x16 rs;
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) {
          if (dt + VD < 16) vread(dt + VD);
          // the 4 reads of dim block dt have completed; up to VD later blocks' may be outstanding
          lgkm_wait(4 * min(VD, 15 - dt));
          order_after(vop[dt % (VD + 1)]);
          oacc[dt] = mfma_fp8_bscaled(vop[dt % (VD + 1)], pb, oacc[dt], psc);
          if (dt == 0) mfma_fp8_v0_bscaled(rs, ones, pb, psc);
          sched_fence();
        }
        asm volatile("" : "+v"(rs));  // read 15 MFMAs later: the sum MFMA has completed
        return rs[0];
      };
      if (__builtin_amdgcn_readfirstlane((int)(k0.cut || k1.cut))) {  // the reference moved
        // earlier tiles were accumulated under the reference before this tile, block 0 under
        // the one before block 1 (whole numbers no greater than the new one, so the scales are
        // exact powers of two in (0, 1]; 1 for the heads that kept their reference). In the
        // first tile of a piece nothing was accumulated before it (the clamp covers the unset
        // reference there).
        const int d_o = min(0, max(-200, (int)(k0.m_old - mref)));
        const int d_0 = min(0, max(-200, (int)(k1.m_old - mref)));
        const float a_o = ldexpf(1.0f, d_o);
#pragma unroll
        for (int d = 0; d < 16; ++d) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {  // in place in the AGPRs that hold O^T
            float x = oacc[d][i], tmp;
            asm volatile(
                "v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\ts_nop 1\n\t"
                "v_accvgpr_write_b32 %0, %1"
                : "+a"(x), "=&v"(tmp)
                : "v"(a_o));
            oacc[d][i] = x;
          }
        }
        asm volatile("s_nop 4" ::: "memory");  // the writes settle before an MFMA reads them
        lsum *= a_o;
        k0.es += d_0;
        if (k0.es < -127) {  // below the smallest E8M0 scale: weight under 2^-119 of the max
          k0.es = 0;
#pragma unroll
          for (int j = 0; j < 4; ++j) k0.w[j] = 0;
        }
      }
      // B operand: bytes 16 b .. 16 b + 15 of lane half h are tokens 32 b + 16 h + 0..15; the
      // scale of k block b comes from lane half b
      const int psc = (hf ? k1.es : k0.es) + 127;
      lsum += pv(i32x8{k0.w[0], k0.w[1], k0.w[2], k0.w[3], k1.w[0], k1.w[1], k1.w[2], k1.w[3]},
                 psc);
      ++t;
      s_cur ^= 1;
    }
    // piece end: request the next piece's Q first (this wave's Q lo area is free), then store
    // this piece's rows through the stage of its last tile
    const int64_t sb = (int64_t)g * F8_SLOTS + slot;
    uint16_t* const rows = complete ? a.out + ((int64_t)cb * a.Hq + head0) * F8_DV
                                    : a.part_o + (sb * a.Hq + head0) * F8_DV;
    float* const lse_at = !complete ? a.part_lse + sb * a.Hq + head
                          : a.seg_lse ? a.seg_lse + (int64_t)cb * a.Hq + head : nullptr;
    const float lse = mref + __log2f(lsum), w = kvs / lsum;
    if (t < t_hi) begin_piece();
    wg_barrier();
    if (complete)
      flush(oacc, rows, lse_at, lse, w, stage(s_cur ^ 1), h16<O_BF16>{});
    else
      flush(oacc, rows, lse_at, lse, w, stage(s_cur ^ 1), h16<true>{});
  }
}

// Online merge of the partial slots of sequence (or segment) v, head `head`, dims d0 .. d0 + 7:
// 0 when v has no tiles, 1 when it lies inside one range (the decode kernel wrote its row), else
// 2 with the running max m, the sum l of 2^(lse - m) and the weighted sum acc (unnormalised).
// v and head are wave-uniform, so the range bookkeeping runs on the scalar unit.
TLM_DEV int f8_merge(const F8Args& a, int v, int head, int d0, float& m, float& l,
                     f32x4 (&acc)[2]) {
  // positions on the cost line (see the prep kernel): v covers [v0, v1), its first tile at
  // v0 + F8_PIECE_COST; range g starts at cost position floor(g V / G)
  const int64_t V = ldc(a.vcu + a.B), v0 = ldc(a.vcu + v), v1 = ldc(a.vcu + v + 1);
  if (v0 == v1) return 0;
  const int64_t G = a.G;
  const int64_t g0 = div_floor((v0 + F8_PIECE_COST + 1) * G - 1, V), g1 = div_floor(v1 * G - 1, V);
  if (g0 == g1) return 1;
  // range starts floor(g V / G) stepped incrementally: floor(g V / G) + V / G, plus one when the
  // remainder (g V) mod G wraps
  const int64_t tq = div_floor(V, G), tr = V - tq * G;
  int64_t s_cur = div_floor(g0 * V, G), r_cur = g0 * V - s_cur * G;  // start of range g, remainder
  auto step = [&](int64_t& st, int64_t& rm) {
    st += tq;
    rm += tr;
    if (rm >= G) {
      rm -= G;
      ++st;
    }
  };
  // range g0 also holds tiles of earlier sequences when it starts before this one: slot 1 there
  const bool first_is_piece = s_cur < v0;
  // Online merge over the ranges in batches of F8_CMB: the lse values and partial outputs of a
  // batch are all requested before any is used, so a call waits for about one memory latency
  // per batch (a sequence spans at most a few ranges at the usual split counts).
  constexpr int F8_CMB = 8;
  m = -INFINITY;
  l = 0.f;
  acc[0] = acc[1] = f32x4{};
  for (int64_t gb = g0; gb <= g1; gb += F8_CMB) {
    float lv[F8_CMB];
    u32x4 pv[F8_CMB];
#pragma unroll
    for (int i = 0; i < F8_CMB; ++i) {
      const int64_t g = gb + i;  // wave-uniform
      lv[i] = -INFINITY;
      pv[i] = u32x4{0u, 0u, 0u, 0u};
      if (g <= g1) {
        int64_t s_next = s_cur, r_next = r_cur;
        step(s_next, r_next);
        if (s_cur != s_next) {  // the range holds tiles
          const int64_t sb = g * F8_SLOTS + ((g == g0 && first_is_piece) ? 1 : 0);
          lv[i] = a.part_lse[sb * a.Hq + head];
          pv[i] = ld_cp<F8_CMB_LOAD_CP>(a.part_o + (sb * a.Hq + head) * F8_DV, 2 * d0);
        }
        s_cur = s_next;
        r_cur = r_next;
      }
    }
    float mb = m;
#pragma unroll
    for (int i = 0; i < F8_CMB; ++i) mb = fmaxf(mb, lv[i]);
    const float r = __builtin_amdgcn_exp2f(m - mb);  // m = -inf on the first batch: r = 0
    l *= r;
    acc[0] *= r;
    acc[1] *= r;
#pragma unroll
    for (int i = 0; i < F8_CMB; ++i) {
      const float w = __builtin_amdgcn_exp2f(lv[i] - mb);  // 0 for an absent range
      l += w;
      acc[0] += bf16x4_to_f32(u32x2{pv[i][0], pv[i][1]}) * w;
      acc[1] += bf16x4_to_f32(u32x2{pv[i][2], pv[i][3]}) * w;
    }
    m = mb;
  }
  return 2;
}

// Merge the partial slots of every sequence that spans more than one range; zero-length
// sequences produce zeros. Thread = (sequence, head, 8 dims); a workgroup covers 4 heads.
template <bool O_BF16>
__global__ __launch_bounds__(256) void mla_fp8_combine(const F8Args a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= (int64_t)a.B * a.Hq) return;
  const int b = (int)(row / a.Hq), head = (int)(row % a.Hq);
  const int d0 = 8 * (threadIdx.x & 63);
  using H = h16<O_BF16>;
  float m, l;
  f32x4 acc[2];
  const int r = f8_merge(a, b, head, d0, m, l, acc);
  if (r == 0) {
    *(u32x4*)(a.out + row * F8_DV + d0) = u32x4{0u, 0u, 0u, 0u};
    return;
  }
  if (r == 1) return;  // whole sequence inside one range: written by the decode kernel
  const float inv = 1.0f / l;
  acc[0] *= inv;
  acc[1] *= inv;
  st_cp<F8_CMB_STORE_CP>(a.out + row * F8_DV, 2 * d0,
                         u32x4{H::pack(acc[0][0], acc[0][1]), H::pack(acc[0][2], acc[0][3]),
                               H::pack(acc[1][0], acc[1][1]), H::pack(acc[1][2], acc[1][3])});
}

// The split programs' combine over segments (example_mla_decode_paged.py:186-221): wave =
// (sequence b, head), thread = 8 dims. Split s is segment b ns + s: its row and lse come from
// the decode kernel (inside one range), from the merge of its pieces, or are -inf and zeros (no
// tokens). Each is stored to Output_partial [b, h, s, :] / glse [b, h, s] in the program's dtype
// (PK as part_store), and Output is the merge of the stored values as read back.
template <int PK, bool O_BF16>
__global__ __launch_bounds__(256) void mla_fp8_segment_combine(const F8Args a, void* glse,
                                                               void* opart, uint16_t* out,
                                                               int ns) {
  using PS = part_store<PK>;
  using HO = h16<O_BF16>;
  const int lane = threadIdx.x & 63;
  const int64_t bh = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (bh >= (int64_t)(a.B / ns) * a.Hq) return;
  const int b = (int)(bh / a.Hq), head = (int)(bh % a.Hq);
  const int d0 = 8 * lane;
  float M = -INFINITY, L = 0.f;
  f32x4 tot[2] = {};
  for (int sp = 0; sp < ns; ++sp) {
    const int v = b * ns + sp;
    float m, l, lse = -INFINITY;
    f32x4 o[2] = {};
    const int r = f8_merge(a, v, head, d0, m, l, o);
    if (r == 1) {
      const int64_t row = (int64_t)v * a.Hq + head;
      lse = a.seg_lse[row];
      const u32x4 x = *(const u32x4*)(a.out + row * F8_DV + d0);
      o[0] = bf16x4_to_f32(u32x2{x[0], x[1]});
      o[1] = bf16x4_to_f32(u32x2{x[2], x[3]});
    } else if (r == 2) {
      lse = m + __log2f(l);
      const float inv = 1.0f / l;
      o[0] *= inv;
      o[1] *= inv;
    }
    if (lane == 0) PS::put_lse(glse, bh * ns + sp, lse);
    f32x4 s0, s1;
    if constexpr (PK == 2) {  // fp32 partials: written once, stored non-temporally (~2.5%)
      __builtin_nontemporal_store(o[0], (f32x4*)opart + ((bh * ns + sp) * F8_DV + d0) / 4);
      __builtin_nontemporal_store(o[1], (f32x4*)opart + ((bh * ns + sp) * F8_DV + d0) / 4 + 1);
      s0 = o[0];
      s1 = o[1];
    } else {
      s0 = PS::put4(opart, (bh * ns + sp) * F8_DV + d0, o[0]);
      s1 = PS::put4(opart, (bh * ns + sp) * F8_DV + d0 + 4, o[1]);
    }
    const float lr = PS::round(lse);  // the stored values, as read back
    if (lr != -INFINITY) {
      const float Mn = fmaxf(M, lr);
      const float c = __builtin_amdgcn_exp2f(M - Mn), w = __builtin_amdgcn_exp2f(lr - Mn);
      L = L * c + w;
      tot[0] = tot[0] * c + s0 * w;
      tot[1] = tot[1] * c + s1 * w;
      M = Mn;
    }
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  *(u32x4*)(out + bh * F8_DV + d0) =
      u32x4{HO::pack(tot[0][0] * inv, tot[0][1] * inv), HO::pack(tot[0][2] * inv, tot[0][3] * inv),
            HO::pack(tot[1][0] * inv, tot[1][1] * inv), HO::pack(tot[1][2] * inv, tot[1][3] * inv)};
}

size_t f8_align(size_t n) { return (n + 255) & ~(size_t)255; }
// tile prefix cu and cost prefix vcu ([B + 1] each), range starts ([G + 1])
size_t f8_cu_bytes(int64_t B, int64_t G) {
  return f8_align((size_t)(B + 1) * 8) + f8_align((size_t)(G + 1) * 4);
}
size_t f8_q_bytes(int64_t B, int64_t Hq) {
  return f8_align((size_t)B * Hq * F8_QROW) + f8_align((size_t)B * Hq * 4);
}

// heads per decode workgroup: 128 (mla_fp8_decode_w32) when Hq is a multiple of 128, else 64
int64_t f8_group_heads(int64_t Hq) { return Hq % W_HEADS == 0 ? W_HEADS : F8_HEADS; }

// ranges per call: B * num_split workgroups shared by the Hq / heads-per-workgroup head groups
int64_t f8_ranges(int64_t B, int64_t Hq, int num_split) {
  return std::max<int64_t>(1, B * num_split / (Hq / f8_group_heads(Hq)));
}

}  // namespace

// Workspace of the fp8 path: tile and cost prefixes and range starts, Q terms, then lse (fp32)
// and O (bf16) partial slots (three slots of Hq x 512 per range).
size_t tlm_mla_fp8_workspace_bytes(int64_t B, int64_t Hq, int num_split) {
  if (Hq % F8_HEADS) return 0;
  const size_t G = (size_t)f8_ranges(B, Hq, num_split);
  return f8_cu_bytes(B, (int64_t)G) + f8_q_bytes(B, Hq) +
         G * F8_SLOTS * (size_t)Hq * (F8_DV * sizeof(uint16_t) + sizeof(float));
}

// Whether the fp8 matrix-core path takes this shape (fp8 KV is checked by the caller).
bool tlm_mla_fp8_applies(int64_t B, int64_t Hq, int64_t page, int64_t max_pages,
                         int64_t kv_stride, int64_t kpe_stride) {
  const int64_t tiles_per_seq = (max_pages * page + F8_TILE - 1) / F8_TILE;
  return Hq % F8_HEADS == 0 && page % F8_TILE == 0 && kv_stride <= (1 << 24) &&
         kpe_stride <= (1 << 24) && B * tiles_per_seq <= INT32_MAX;
}

// Workspace of the split programs' path (tlm_mla_fp8_launch_segments): the fp8 path's layout over
// B * num_split segments and the ranges of `par` (Q terms still per sequence), then each
// segment's bf16 rows and fp32 lse.
size_t tlm_mla_fp8_segments_workspace_bytes(int64_t B, int64_t Hq, int num_split, int par) {
  if (Hq % W_HEADS) return 0;
  const int64_t Bv = B * num_split;
  const size_t G = (size_t)f8_ranges(B, Hq, par);
  return f8_cu_bytes(Bv, (int64_t)G) + f8_q_bytes(B, Hq) +
         G * F8_SLOTS * (size_t)Hq * (F8_DV * sizeof(uint16_t) + sizeof(float)) +
         f8_align((size_t)Bv * Hq * F8_DV * sizeof(uint16_t)) + f8_align((size_t)Bv * Hq * 4);
}

namespace {

F8Args f8_args(const void* q, const void* q_pe, int64_t q_stride, int64_t q_pe_stride,
               const void* kv, const void* k_pe, int64_t kv_stride, int64_t kpe_stride,
               int64_t kv_rows, const int32_t* block_table, const int32_t* seqlens, int64_t page,
               int64_t max_pages, float score_scale, const float* kv_scale) {
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
  a.page = (int)page;
  a.max_pages = (int)max_pages;
  a.lmax = (int)(max_pages * page);
  a.score_scale = score_scale;
  a.kv_scale = kv_scale;
  a.nsp = 1;
  a.seg_lse = nullptr;
  return a;
}

// Prep, decode and combine over B * nsp segments (nsp splits of each of B sequences) cut into G
// ranges; the workspace starts with the prefixes and range starts, then the Q terms of the B
// sequences and the partial slots of the G ranges.
int f8_run(F8Args& a, void* ws, int64_t B, int64_t Hq, int nsp, int64_t G, bool q_bf16,
           bool o_bf16, hipStream_t st, bool combine = true) {
  const int64_t Bv = B * nsp;
  a.cu = (int32_t*)ws;
  a.vcu = a.cu + (Bv + 1);
  a.range_t = (int32_t*)((char*)ws + f8_align((size_t)(Bv + 1) * 8));
  a.qsplit = (uint8_t*)ws + f8_cu_bytes(Bv, G);
  a.qexp = (int32_t*)(a.qsplit + f8_align((size_t)B * Hq * F8_QROW));
  a.part_lse = (float*)((char*)ws + f8_cu_bytes(Bv, G) + f8_q_bytes(B, Hq));
  a.part_o = (uint16_t*)(a.part_lse + G * F8_SLOTS * Hq);
  a.B = (int)Bv;
  a.Hq = (int)Hq;
  a.G = (int)G;
  a.nsp = nsp;
  const int HG = (int)(Hq / f8_group_heads(Hq));
  const int nq = (int)((B * Hq + 3) / 4);
  if (q_bf16)
    mla_fp8_prep<true><<<nq + 1, 256, 0, st>>>(a, nq);
  else
    mla_fp8_prep<false><<<nq + 1, 256, 0, st>>>(a, nq);
  TLM_LAUNCH_CHECK("tlm_mla_decode (fp8 prep)");
  const dim3 grid((unsigned)(((G + 7) / 8) * 8 * HG));
  if (f8_group_heads(Hq) == W_HEADS) {
    if (o_bf16)
      mla_fp8_decode_w32<true><<<grid, 256, 0, st>>>(a);
    else
      mla_fp8_decode_w32<false><<<grid, 256, 0, st>>>(a);
  } else if (o_bf16) {
    mla_fp8_decode<true><<<grid, 512, 0, st>>>(a);
  } else {
    mla_fp8_decode<false><<<grid, 512, 0, st>>>(a);
  }
  TLM_LAUNCH_CHECK("tlm_mla_decode (fp8 decode)");
  if (!combine) return TLM_OK;
  const dim3 cgrid((unsigned)((Bv * Hq + 3) / 4));
  if (o_bf16) mla_fp8_combine<true><<<cgrid, 256, 0, st>>>(a);
  else mla_fp8_combine<false><<<cgrid, 256, 0, st>>>(a);
  TLM_LAUNCH_CHECK("tlm_mla_decode (fp8 combine)");
  return TLM_OK;
}

}  // namespace

// Returns TLM_EUNSUPPORTED (launching nothing) when the shape is outside this kernel's domain.
int tlm_mla_fp8_launch(const void* q, const void* q_pe, int64_t q_stride, int64_t q_pe_stride,
                       const void* kv, const void* k_pe, int64_t kv_stride, int64_t kpe_stride,
                       int64_t kv_rows, const int32_t* block_table, const int32_t* seqlens,
                       void* o, void* ws, int64_t B, int64_t Hq, int64_t page, int64_t max_pages,
                       int num_split, float score_scale, const float* kv_scale, bool q_bf16,
                       bool o_bf16, void* stream) {
  if (!tlm_mla_fp8_applies(B, Hq, page, max_pages, kv_stride, kpe_stride))
    return TLM_EUNSUPPORTED;
  F8Args a = f8_args(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride, kpe_stride, kv_rows,
                     block_table, seqlens, page, max_pages, score_scale, kv_scale);
  a.out = (uint16_t*)o;
  // num_split sets the ranges (B * num_split workgroups over all head groups), not a partition
  return f8_run(a, ws, B, Hq, 1, f8_ranges(B, Hq, num_split), q_bf16, o_bf16,
                (hipStream_t)stream);
}

// The split programs' partition (num_split segments per sequence, example_mla_decode_paged.py:
// 140-144 with block_N = 64) on the 128-head decode, balanced over f8_ranges(B, Hq, par) ranges,
// then mla_fp8_segment_combine: glse / o_partial of p_dtype (TLM_F16 / TLM_BF16 / TLM_F32) and
// Output o. Returns TLM_EUNSUPPORTED (launching nothing) outside this path's domain.
int tlm_mla_fp8_launch_segments(const void* q, const void* q_pe, int64_t q_stride,
                                int64_t q_pe_stride, const void* kv, const void* k_pe,
                                int64_t kv_stride, int64_t kpe_stride, int64_t kv_rows,
                                const int32_t* block_table, const int32_t* seqlens, void* ws,
                                int64_t B, int64_t Hq, int64_t page, int64_t max_pages,
                                int num_split, int par, float score_scale,
                                const float* kv_scale, bool q_bf16, void* glse, void* o_partial,
                                int p_dtype, void* o, bool o_bf16, void* stream) {
  if (!tlm_mla_fp8_applies(B, Hq, page, max_pages, kv_stride, kpe_stride) || Hq % W_HEADS ||
      num_split < 1 || B * num_split > INT32_MAX / 2)
    return TLM_EUNSUPPORTED;
  F8Args a = f8_args(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride, kpe_stride, kv_rows,
                     block_table, seqlens, page, max_pages, score_scale, kv_scale);
  const int64_t Bv = B * num_split;
  const int64_t G = f8_ranges(B, Hq, par);
  // segments inside one range leave their row (bf16) and lse here for the segment combine
  char* tail = (char*)ws + f8_cu_bytes(Bv, G) + f8_q_bytes(B, Hq) +
               G * F8_SLOTS * (size_t)Hq * (F8_DV * sizeof(uint16_t) + sizeof(float));
  a.out = (uint16_t*)tail;
  a.seg_lse = (float*)(tail + f8_align((size_t)Bv * Hq * F8_DV * sizeof(uint16_t)));
  hipStream_t st = (hipStream_t)stream;
  const int rc = f8_run(a, ws, B, Hq, num_split, G, q_bf16, true, st, false);
  if (rc) return rc;
  const dim3 cgrid((unsigned)((B * Hq + 3) / 4));
  auto comb = [&](auto kern) {
    kern<<<cgrid, 256, 0, st>>>(a, glse, o_partial, (uint16_t*)o, num_split);
  };
  if (p_dtype == TLM_F32)
    o_bf16 ? comb(mla_fp8_segment_combine<2, true>) : comb(mla_fp8_segment_combine<2, false>);
  else if (p_dtype == TLM_BF16)
    o_bf16 ? comb(mla_fp8_segment_combine<1, true>) : comb(mla_fp8_segment_combine<1, false>);
  else
    o_bf16 ? comb(mla_fp8_segment_combine<0, true>) : comb(mla_fp8_segment_combine<0, false>);
  TLM_LAUNCH_CHECK("tlm_mla_decode (fp8 segment combine)");
  return TLM_OK;
}
