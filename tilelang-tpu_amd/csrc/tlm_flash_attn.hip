// FlashAttention forward (BSHD) on gfx950 MFMA.
//
// Reference program: tpu_demo/flashattn/tpu_test_flashattn_bf16.py:14-135 — per Q tile, loop over
// KV tiles: S = Q K^T (ppl_gemm transpose_B), online softmax (m = rowmax, alpha = exp((m_prev-m)*sc),
// P = exp((S-m)*sc), l = l*alpha + rowsum(P)), P cast to the input dtype, O = O*alpha + P V,
// finally O / l. Causal keeps key j <= query i (element mask of ref_program :171-182 and of the
// upstream example_mha_fwd_bshd.py:50-53).
//
// Kernels:
//   * fa_fwd_pp (head dim 128, the config kernel): workgroup = 8 waves = 256 queries of one
//     (batch, head); wave w owns a 32-query block and computes S^T = K Q^T and O^T = V^T P^T on
//     v_mfma_f32_16x16x32 as two 16-query tiles (each lane holds 16 keys of each of its two
//     queries; the softmax statistics combine the four lane groups with xor-16 / xor-32
//     exchanges). P^T goes from the S^T accumulator to the PV B operand in registers; V^T comes
//     from the row-major V tile through ds_read_b64_tr_b16; Q stays in VGPRs. K and V tiles of 64
//     keys stream through 4-stage LDS rings fed by buffer_load ... lds (the tile two steps ahead
//     is loaded during the current step; descriptor bounds zero the keys past the sequence).
//     Waves w and w + 4 share a SIMD and run one phase apart (ping-pong): while one issues its
//     QK + PV MFMAs the other runs its softmax on the VALU. Softmax with a lazy running max: a
//     tile is exponentiated against the current maximum and only redone (maximum raised, O and l
//     rescaled) when its P sum leaves the 16-bit P range. Causal workgroups take two query tiles
//     of one head (nqt - 1 - s and s), so every workgroup does the same number of key tiles;
//     workgroup ids are regrouped so all query tiles of a (batch, head) run on one XCD.
//   * fa_fwd (head dim 64): 8 waves x 32 queries on v_mfma_f32_32x32x16 (S^T = K Q^T, one query
//     and 16 keys per lane), K/V tiles double-buffered in padded LDS with register staging; the
//     non-causal form uses the same lazy-max softmax, the causal form a per-tile maximum.
//   * fa_fwd_generic (other head dims up to 256, fp32 output at D = 64): one query per lane, q
//     and O in VGPRs, per-key online softmax, P rounded to the input type.
// Softmax runs in the exp2 domain with sm_scale * log2(e) folded into one fma.
#include "tlm_common.h"

#include <algorithm>
#include <type_traits>
#include <utility>

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int FA_WAVES = 8;
constexpr int BQ = 32 * FA_WAVES;  // queries per workgroup
constexpr int BKV = 64;            // keys per tile

// Query and key rows of batch b. Dense (cu_q == nullptr): every sequence holds s_q queries and
// s_k keys, starting at rows b s_q and b s_k. Variable length: cu_q / cu_k are the [B + 1] prefix
// sums of the sequence lengths (examples/flash_attention/example_mha_fwd_varlen.py:267-276),
// s_q / s_k the row counts of Q / O and K / V; a sequence whose rows fall outside them is taken
// as empty, so bad offsets never address memory outside the tensors.
// Element strides: tq / tk between consecutive tokens of Q, O / K, V, hq / hk between heads.
// Sequence-major [B, S, H, D] (and the unpadded [T, H, D]): tq = H D, hq = D. Head-major
// [B, H, S, D] (examples/flash_attention/example_mha_fwd_bhsd.py:32-33): tq = D, hq = S_q D.
// Either way batch b's rows start at element (first row) H D.
struct SeqMap {
  const int* cu_q;
  const int* cu_k;
  int s_q, s_k;
  int64_t tq, tk, hq, hk;
};
struct SeqRange {
  int64_t q0, k0;  // first row of the sequence's queries / keys
  int nq, nk;      // their counts
};
TLM_DEV SeqRange seq_range(const SeqMap& m, int b) {
  if (m.cu_q == nullptr) return {(int64_t)b * m.s_q, (int64_t)b * m.s_k, m.s_q, m.s_k};
  const int q0 = m.cu_q[b], q1 = m.cu_q[b + 1], k0 = m.cu_k[b], k1 = m.cu_k[b + 1];
  const bool ok = 0 <= q0 && q0 <= q1 && q1 <= m.s_q && 0 <= k0 && k0 <= k1 && k1 <= m.s_k;
  if (!ok) return {0, 0, 0, 0};
  return {q0, k0, q1 - q0, k1 - k0};
}

TLM_DEV s16x4 lds_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

// Key split of the split-KV inference program (examples/flash_attention/example_mha_inference.py:
// 98-160): program split s covers keys [s per, (s + 1) per) of its sequence; each is cut into r
// internal parts of per_i keys (the last may be shorter or empty) so the launch fills the chip.
// Internal split si = s r + j writes its normalised fp32 output to O [B][S_q][H][nsi][D] and its
// log2 sum-exp (scaled-score units; -inf for no keys) to lse [B][S_q][H][nsi].
struct FaSplit {
  float* lse;
  int nsi, r, per, per_i;
};
TLM_DEV SeqRange split_keys(SeqRange sr, const FaSplit& sp, int si) {
  const int s = si / sp.r, j = si % sp.r;
  sr.k0 += (int64_t)s * sp.per + (int64_t)j * sp.per_i;
  sr.nk = max(0, min(sp.per_i, sp.per - j * sp.per_i));
  return sr;
}

template <bool BF16>
struct fa_mma;
template <>
struct fa_mma<false> {
  typedef f16x8 v8;
  static TLM_DEV f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct fa_mma<true> {
  typedef bf16x8 v8;
  static TLM_DEV f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <bool BF16>
struct fa_mma16;
template <>
struct fa_mma16<false> {
  typedef f16x8 v8;
  static TLM_DEV f32x4 mma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct fa_mma16<true> {
  typedef bf16x8 v8;
  static TLM_DEV f32x4 mma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <bool BF16, bool CAUSAL, int D>
__global__ __launch_bounds__(64 * FA_WAVES, 1) void fa_fwd(const uint16_t* __restrict__ Q,
                                                          const uint16_t* __restrict__ K,
                                                          const uint16_t* __restrict__ V,
                                                          uint16_t* __restrict__ O, int B, int S,
                                                          int H, int Hkv, float scale_log2,
                                                          SeqMap sm) {
  using MT = fa_mma<BF16>;
  using v8 = typename MT::v8;
  using HH = h16<BF16>;
  constexpr int KP = D + 8;    // K tile pitch (halves): conflict-free 16-byte row reads
  constexpr int VP = D + 16;   // V tile pitch: conflict-free transpose reads
  constexpr int DS = D / 16;   // k-substeps of S^T
  constexpr int DT = D / 32;   // 32-wide d tiles of O^T
  constexpr int CH = D / 8;    // 16-byte chunks per row
  constexpr int LD_ITERS = BKV * CH / (64 * FA_WAVES);  // K (and V) vectors per thread per tile
  constexpr int OP = D + 8;    // epilogue staging pitch
  constexpr int SMEM = 2 * BKV * (KP + VP);
  static_assert(LD_ITERS >= 1, "tile too small for the thread count");
  static_assert(BQ * OP <= SMEM, "epilogue staging must fit in the K/V buffers");
  __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM];
  uint16_t* sK = smem;                  // [2][BKV][KP]
  uint16_t* sV = smem + 2 * BKV * KP;   // [2][BKV][VP]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nqt = (S + BQ - 1) / BQ;
  const int lin = blockIdx.x;
  const int qt = nqt - 1 - lin / (B * H);  // heaviest (last) query tiles first
  const int bh = lin % (B * H);
  const int b = bh / H, h = bh % H;
  const int q0 = qt * BQ;
  // S counts the grid's query tiles; the sequence's own counts are Sq, Sk (causal: query i sees
  // keys j <= i + Sk - Sq)
  const SeqRange sr = seq_range(sm, b);
  const int Sq = sr.nq, Sk = sr.nk, coff = Sk - Sq;
  if (q0 >= Sq) return;  // whole workgroup, before any barrier
  const int64_t row_stride = sm.tq;  // elements between consecutive tokens (Q, O)
  const int64_t kv_stride = sm.tk;   // K, V: Hkv heads, query head h reads h / (H/Hkv)
  const int hk = h / (H / Hkv);
  const int64_t head = sr.q0 * H * D + h * sm.hq;
  const uint16_t* Qb = Q + head;
  const uint16_t* Kb = K + sr.k0 * Hkv * D + hk * sm.hk;
  const uint16_t* Vb = V + sr.k0 * Hkv * D + hk * sm.hk;

  const int ql = lane & 31, g = lane >> 5;
  const int qw0 = q0 + 32 * wave;  // first query of this wave
  const int my_q = qw0 + ql;

  // Q^T operand: lane holds query my_q, d = 16*ds + 8*g .. +7
  v8 qreg[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    u32x4 v = {0, 0, 0, 0};
    if (my_q < Sq) v = *(const u32x4*)(Qb + (int64_t)my_q * row_stride + 16 * ds + 8 * g);
    qreg[ds] = __builtin_bit_cast(v8, v);
  }

  const int kv_end = CAUSAL ? max(0, min(Sk, q0 + BQ + coff)) : Sk;
  const int nblk = (kv_end + BKV - 1) / BKV;
  const int wave_qmax = min(qw0 + 31, Sq - 1);  // < qw0 when the whole wave is past Sq

  u32x4 rk[LD_ITERS], rv[LD_ITERS];
  auto load_tile = [&](int j) {
#pragma unroll
    for (int p = 0; p < LD_ITERS; ++p) {
      const int idx = tid + p * 64 * FA_WAVES;
      const int r = idx / CH, c = (idx % CH) * 8;
      const int key = j * BKV + r;
      if (key < Sk) {
        rk[p] = *(const u32x4*)(Kb + (int64_t)key * kv_stride + c);
        rv[p] = *(const u32x4*)(Vb + (int64_t)key * kv_stride + c);
      } else {
        rk[p] = u32x4{0, 0, 0, 0};
        rv[p] = u32x4{0, 0, 0, 0};
      }
    }
  };
  auto store_tile = [&](int stage) {
#pragma unroll
    for (int p = 0; p < LD_ITERS; ++p) {
      const int idx = tid + p * 64 * FA_WAVES;
      const int r = idx / CH, c = (idx % CH) * 8;
      *(u32x4*)(sK + stage * BKV * KP + r * KP + c) = rk[p];
      *(u32x4*)(sV + stage * BKV * VP + r * VP + c) = rv[p];
    }
  };

  f32x16 oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = f32x16{};
  float m_run = -INFINITY, l_part = 0.f;

  // transpose-read lane roles for V^T: 16-lane group hh, lane jj
  const int hh = lane >> 4, jj = lane & 15;

  if (nblk > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int j = 0; j < nblk; ++j) {
    const int cur = j & 1;
    const bool has_next = j + 1 < nblk;
    if (has_next) load_tile(j + 1);
    const int k0 = j * BKV;
    const bool active = (qw0 < Sq) && (!CAUSAL || k0 <= wave_qmax + coff);
    if (active) {
      const uint16_t* kt = sK + cur * BKV * KP;
      const uint16_t* vt = sV + cur * BKV * VP;
      // S^T[key][query] for two 32-key tiles
      f32x16 sacc[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        sacc[t] = f32x16{};
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
          const v8 a = *(const v8*)(kt + (32 * t + ql) * KP + 16 * ds + 8 * g);
          sacc[t] = MT::mma(a, qreg[ds], sacc[t]);
        }
      }
      v8 pb[2][2];
      if constexpr (!CAUSAL) {
        // mask (keys of this lane: 32t + 8(i/4) + 4g + i%4), then P = 2^(s sc - m) against the
        // running m without the tile's max (a lazy max): only when the lane's P sum of the tile
        // leaves P_LIMIT (or is not finite: the first tile, where m = -inf) is the tile redone
        // with m raised to its max and O, l rescaled. The common factor cancels in O / l, so the
        // result is the same softmax at about 3.5 VALU operations per score instead of 6.5 (no
        // separate scale, max or per-tile O rescale). P_LIMIT keeps every P in range of the 16-bit
        // type (fp16: P <= 2^15; bf16: 2^64) and O, l far from fp32 overflow. Non-causal only
        // (+11% at B 8, H 32, S 4096, fp16): the causal kernel measured 5% slower with it, both
        // at 143 VGPRs (one workgroup per CU) and forced to 128 (two), so it keeps the per-tile
        // max below.
        constexpr float P_LIMIT = BF16 ? 18446744073709551616.0f : 32768.0f;
        const bool need_mask = (CAUSAL && k0 + BKV - 1 > qw0 + coff) || (k0 + BKV > Sk);
        if (need_mask) {
  #pragma unroll
          for (int t = 0; t < 2; ++t)
  #pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int key = k0 + 32 * t + 8 * (i >> 2) + 4 * g + (i & 3);
              if (key >= Sk || (CAUSAL && key > my_q + coff)) sacc[t][i] = -INFINITY;
            }
        }
        auto exp_tile = [&](float nb) __attribute__((always_inline)) {  // fills pb, returns the lane's P sum
          float s0 = 0.f, s1 = 0.f;
  #pragma unroll
          for (int t = 0; t < 2; ++t)
  #pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
              u32x4 pk;
  #pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float p0 = fast_exp2(__builtin_fmaf(sacc[t][8 * s2 + 2 * e], scale_log2, nb));
                const float p1 =
                    fast_exp2(__builtin_fmaf(sacc[t][8 * s2 + 2 * e + 1], scale_log2, nb));
                if (e & 1) s1 += p0 + p1; else s0 += p0 + p1;
                pk[e] = HH::pack(p0, p1);
              }
              pb[t][s2] = __builtin_bit_cast(v8, pk);
            }
          return s0 + s1;
        };
        // the first tile (m = -inf) always needs its max: skip the exponentials it would redo
        float psum = j > 0 ? exp_tile(-m_run) : 0.f;
        if (j == 0 || __builtin_amdgcn_ballot_w64(!(psum <= P_LIMIT))) {  // rare: raise m
          float mx = -INFINITY;
  #pragma unroll
          for (int t = 0; t < 2; ++t)
  #pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[t][i]);
          mx = fmaxf(mx, __shfl_xor(mx, 32, 64));  // the query's other 32 keys
          const float m_new = fmaxf(m_run, mx * scale_log2);
          const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run - m_new);
          m_run = m_new;
          l_part *= alpha;
  #pragma unroll
          for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
          psum = exp_tile(m_new == -INFINITY ? 0.f : -m_new);
        }
        l_part += psum;
      } else {
        // scale, mask, row max (keys of this lane: 32t + 8(i/4) + 4g + i%4)
        const bool need_mask = (CAUSAL && k0 + BKV - 1 > qw0 + coff) || (k0 + BKV > Sk);
        float mloc = -INFINITY;
  #pragma unroll
        for (int t = 0; t < 2; ++t)
  #pragma unroll
          for (int i = 0; i < 16; ++i) {
            float x = sacc[t][i] * scale_log2;
            if (need_mask) {
              const int key = k0 + 32 * t + 8 * (i >> 2) + 4 * g + (i & 3);
              if (key >= Sk || (CAUSAL && key > my_q + coff)) x = -INFINITY;
            }
            sacc[t][i] = x;
            mloc = fmaxf(mloc, x);
          }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        const float m_new = fmaxf(m_run, mloc);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = fast_exp2(m_run - m_use);
        m_run = m_new;
        float psum = 0.f;
  #pragma unroll
        for (int t = 0; t < 2; ++t)
  #pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            u32x4 pk;
  #pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float p0 = fast_exp2(sacc[t][8 * s2 + 2 * e] - m_use);
              const float p1 = fast_exp2(sacc[t][8 * s2 + 2 * e + 1] - m_use);
              psum += p0 + p1;
              pk[e] = HH::pack(p0, p1);
            }
            pb[t][s2] = __builtin_bit_cast(v8, pk);
          }
        l_part = l_part * alpha + psum;
  #pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
      }
      // O^T += V^T P^T
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int base = 32 * t + 16 * s2 + 4 * (hh >> 1) + (jj >> 2);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const uint16_t* p = vt + base * VP + 32 * dt + 16 * (hh & 1) + 4 * (jj & 3);
            const s16x4 lo = lds_tr16(p), hi = lds_tr16(p + 8 * VP);
            typedef short s16x8 __attribute__((ext_vector_type(8)));
            const s16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            oacc[dt] = MT::mma(__builtin_bit_cast(v8, av), pb[t][s2], oacc[dt]);
          }
        }
    }
    if (has_next) store_tile(cur ^ 1);
    __syncthreads();
  }

  // normalise and write: lane holds O^T[d = 32dt + 8(i/4) + 4g + i%4][query my_q]
  const float l_tot = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  uint16_t* stage = smem + wave * 32 * OP;  // [32 queries][OP]
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = 32 * dt + 8 * (i >> 2) + 4 * g + (i & 3);
      stage[ql * OP + d] = (uint16_t)HH::from_f32(oacc[dt][i] * inv);
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  uint16_t* Ob = O + head;
#pragma unroll
  for (int it = 0; it < 32 * CH / 64; ++it) {
    const int idx = lane + 64 * it;
    const int r = idx / CH, c = (idx % CH) * 8;
    const int q = qw0 + r;
    if (q < Sq) *(u32x4*)(Ob + (int64_t)q * row_stride + c) = *(const u32x4*)(stage + r * OP + c);
  }
}

// ---------------------------------------------------------------------------------------------
// Head dim 128: ping-pong kernel.
//
//   * workgroup = 8 waves = 256 queries of one (batch, head); a wave owns one 32-query block and
//     computes S^T = K Q^T and O^T = V^T P^T with v_mfma_f32_16x16x32 (two 16-query tiles; Q^T
//     in VGPRs, P^T straight from the S^T accumulator). A lane holds 16 keys of each of its two
//     queries, so the softmax statistics combine the four lane groups with xor-16 and xor-32
//     exchanges. The 16x16 shape draws less power per FLOP than 32x32x16 (a higher sustained
//     clock: +3.6% at S 2048 non-causal);
//   * the waves form two groups of four (one wave of each group per SIMD) that run one phase
//     apart: while one group issues MFMAs (QK of tile j and PV of tile j-1: 32 MFMAs per wave, at
//     raised wave priority) the other runs the softmax of its tile on the VALU, so each SIMD's
//     matrix core and VALU are busy at the same time. Each half-step ends with a workgroup
//     barrier. (Interleaving each wave's own softmax into its MFMA stream instead, one piece of
//     the next tile's softmax after each PV MFMA, measured 7% slower with 8 waves of 32 queries
//     and 25-33% slower with 4 waves of 64 queries, where one wave per SIMD cannot cover its own
//     LDS and VALU latencies);
//   * K and V tiles (64 keys x 128 dims, 16 KB each) stream into 4-stage LDS rings through
//     buffer_load ... lds (16 bytes per lane, no VGPR staging). Tile j + 2 is loaded during step j;
//     the buffer descriptor of a tile ends at its last valid key, so keys >= S read as zeros;
//   * LDS layout: rows of 256 bytes, 16-byte chunk c of key row r stored at chunk c ^ (r & 15) for
//     K (the ds_read_b128 row reads of 16 lanes hit 16 distinct chunks) and c ^ 2 (r & 7) for V
//     (the ds_read_b64_tr_b16 reads of 32 lanes cover 8 key rows x 2 chunks);
//   * online softmax with a lazy running max: a tile is exponentiated against the current m
//     without computing its max; only when its P sum leaves the safe range (bf16 2^64, fp16 2^15;
//     also the first tile, where m = -inf) is it redone with m raised to the tile max and O, l
//     rescaled. The result is the same softmax (the common factor cancels in O / l) at about 3.5
//     VALU operations per score (fma, exp2, add into the fp32 row sum, half a pack). v_dot2 is
//     avoided on purpose: it does not overlap with the MFMAs of the other wave on the SIMD;
//   * query blocks are assigned so that the two waves sharing a SIMD hold blocks b and 7 - b
//     (equal causal work per SIMD), and workgroup ids are regrouped so that one XCD runs all query
//     tiles of a (batch, head) together, heaviest first: its K/V tiles are then read from that
//     XCD's L2 by up to 16 workgroups at about the same time.
constexpr int PP_D = 128;
constexpr int PP_BQ = 256;                        // queries per workgroup
constexpr int PP_KV = 64;                         // keys per tile
constexpr int PP_TILE = PP_KV * PP_D * 2;         // bytes of one K or V tile
constexpr int PP_NST = 4;                         // ring stages (tiles j-1 .. j+2 live in step j)
constexpr int PP_VRING = PP_NST * PP_TILE;        // V ring follows the K ring
constexpr int PP_SMEM = 2 * PP_NST * PP_TILE;     // 128 KB
constexpr int PP_OP = PP_D + 8;                   // epilogue staging pitch (halves)
constexpr int PP_RSRC_WORD3 = 0x00020000;         // raw buffer, 32-bit data format
// Cache policy of the K / V LDS-DMA loads (st_cp bits). Plain: the query tiles of one K / V head
// re-read its tiles from L2. Non-temporal loads measured 4-5% slower for causal and, for full
// attention, 1-2% faster at S 2048, neutral for head-major and grouped-query, 3-4% slower for
// ragged batches (1,038-1,044 against 1,069-1,084 TFLOP/s), whose counted fetches rose from
// 1.12 to 1.77 times the algorithmic bytes (grouped-query: 1.88 to 2.45). Split-KV parts whose
// tiles are each read by one workgroup (one query tile, no shared K / V heads) load them
// non-temporally: a stand-alone copy of that read pattern streamed 6.2 against 5.1 TB/s.
constexpr int PP_KV_CP = CP_PLAIN;
static_assert(8 * 32 * PP_OP * 2 <= PP_SMEM, "epilogue staging must fit in the rings");

#define TLM_INLINE __attribute__((always_inline))

template <typename F, int... I>
TLM_DEV void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
TLM_DEV void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// LDS reads as inline asm with an immediate offset: compiler-generated LDS reads may be made to
// wait for all outstanding LDS-DMA loads (including prefetches of later tiles). Their completion
// is awaited explicitly with lgkm_wait.
template <int OFF>
TLM_DEV u32x4 ds_b128(uint32_t a) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF) : "memory");
  return r;
}
template <int OFF>
TLM_DEV u32x2 ds_tr16(uint32_t a) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF) : "memory");
  return r;
}
template <int N>
TLM_DEV void lgkm_wait() {  // s_waitcnt lgkmcnt(N)
  static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
  __builtin_amdgcn_s_waitcnt(0xc07f | (N << 8));
}
template <int N>
TLM_DEV void vm_wait() {  // s_waitcnt vmcnt(N)
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x3f70 | (N & 15) | ((N >> 4) << 14));
}
TLM_DEV void order_after(u32x4& a) { asm volatile("" : "+v"(a)); }
TLM_DEV uint32_t lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// Workgroup barrier at a phase boundary: this wave's LDS reads have completed; sched_barrier
// keeps the scheduler from moving MFMAs (register-only instructions) across it.
TLM_DEV void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// NT (split parts whose K / V tiles are each read by one workgroup): non-temporal K / V loads.
template <bool BF16, bool CAUSAL, bool OUT32, bool SPLIT = false, bool NT = false>
__global__ __launch_bounds__(512, 1) void fa_fwd_pp(const uint16_t* __restrict__ Q,
                                                   const uint16_t* __restrict__ K,
                                                   const uint16_t* __restrict__ V,
                                                   void* __restrict__ O, int B, int S, int H,
                                                   int Hkv, float sc, SeqMap sm, FaSplit sp) {
  static_assert(!SPLIT || (OUT32 && !CAUSAL), "split parts are non-causal with fp32 output");
  using MT = fa_mma16<BF16>;
  using v8 = typename MT::v8;
  using HH = h16<BF16>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[PP_SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, wl = wave & 3;
  // query block of the wave (waves w and w + 4 share a SIMD). Causal: the pairs (0, 7), (2, 5),
  // (4, 3), (6, 1) give every SIMD the same key count. Otherwise wave w takes block w, so a tile
  // of at most 128 queries (split inference, ragged tails) has all its working waves in group 0:
  // a step is then one MFMA phase and one softmax phase instead of two of each.
  const int blk = CAUSAL ? (grp == 0 ? 2 * wl : 7 - 2 * wl) : wave;

  // workgroup -> (batch, head, slot). Workgroup ids go round-robin over the 8 XCDs; each XCD
  // takes whole K/V heads: all query tiles of the G = H / Hkv query heads that read one K/V head
  // run there together, so their K/V tiles come from that XCD's L2. Causal: slot s holds query
  // tiles nqt - 1 - s and s of one head, (nqt - s) + (s + 1) key tiles together, so every
  // workgroup carries the same work. The dispatcher gives every CU the same number of workgroups
  // whatever their length (measured: 16 per CU at B 8, H 32, S 4096), so workgroups of unequal
  // work leave CUs idle; one tile per workgroup kept them busy 79% of the time.
  const int nqt = (S + PP_BQ - 1) / PP_BQ;
  const int nslot = CAUSAL ? (nqt + 1) / 2 : nqt;
  const int G = H / Hkv;
  int lin = blockIdx.x;
  int b, h, slot, si = 0;
  if constexpr (SPLIT) {  // workgroup = (internal split, batch, head, query tile)
    si = lin % sp.nsi;
    lin /= sp.nsi;
  }
  if (!SPLIT && (B * Hkv) % 8 == 0) {
    const int xcd = lin & 7, s = lin >> 3;
    const int per = nslot * G;  // workgroups per K/V head
    const int kvh = (s / per) * 8 + xcd, rem = s % per;
    slot = rem % nslot;
    b = kvh / Hkv;
    h = (kvh % Hkv) * G + rem / nslot;
  } else {
    const int bh = lin / nslot;
    slot = lin % nslot;
    b = bh / H;
    h = bh % H;
  }
  // S counts the query tiles of the grid; the sequence's own query and key counts are Sq, Sk.
  // Causal: query i sees keys j <= i + (Sk - Sq) (bottom-right aligned; 0 offset when dense).
  SeqRange sr = seq_range(sm, b);
  if constexpr (SPLIT) sr = split_keys(sr, sp, si);
  const int n_items = CAUSAL && 2 * slot != nqt - 1 ? 2 : 1;
  for (int item = 0; item < n_items; ++item) {
  const int qt = CAUSAL && item == 0 ? nqt - 1 - slot : slot;
  [&]() TLM_INLINE {  // one query tile; a return ends the tile
  const int q0 = qt * PP_BQ;
  const int Sq = sr.nq, Sk = sr.nk, coff = Sk - Sq;
  if (q0 >= Sq) return;  // whole workgroup
  const int64_t rs = sm.tq;     // elements between consecutive tokens of Q, O
  const int64_t rs_kv = sm.tk;  // ... of K, V
  const int64_t head = sr.q0 * H * PP_D + h * sm.hq;
  const int64_t head_kv = sr.k0 * Hkv * PP_D + (h / G) * sm.hk;
  const uint16_t* Qb = Q + head;

  const int n_all = (Sk + PP_KV - 1) / PP_KV;
  const int kv_vis = q0 + PP_BQ + coff;  // keys visible to the workgroup's last query row, + 1
  const int n = CAUSAL ? (kv_vis <= 0 ? 0 : min(n_all, (kv_vis + PP_KV - 1) / PP_KV))
                       : n_all;  // key tiles of the workgroup
  const int qb0 = q0 + 32 * blk;  // first query of the wave
  const int w_last = qb0 + 31 + coff;  // last key visible to the wave
  const int nw = qb0 >= Sq ? 0 : (CAUSAL ? (w_last < 0 ? 0 : min(n, w_last / PP_KV + 1)) : n);

  // v_mfma_f32_16x16x32 roles: lane l works on column (query) l % 16 of a 16-wide tile and on
  // k group g = l / 16; the wave's 32 queries are two 16-query tiles qq
  const int ql = lane & 15, g = lane >> 4;
  const int my_q[2] = {qb0 + ql, qb0 + 16 + ql};

  // Q^T operand (B of S^T = K Q^T): lane holds query my_q[qq], d = 32 dk + 8 g .. + 7
  v8 qreg[2][PP_D / 32];
#pragma unroll
  for (int qq = 0; qq < 2; ++qq)
#pragma unroll
    for (int dk = 0; dk < PP_D / 32; ++dk) {
      u32x4 v = {0, 0, 0, 0};
      if (my_q[qq] < Sq) v = *(const u32x4*)(Qb + (int64_t)my_q[qq] * rs + 32 * dk + 8 * g);
      qreg[qq][dk] = __builtin_bit_cast(v8, v);
    }

  // ---- LDS-DMA: group 0 fills K tiles, group 1 V tiles; wave wl writes rows 16 wl .. 16 wl + 15
  // (4 instructions of 4 rows x 16 chunks). Lane -> (row, stored chunk p) fetches chunk p ^ swz.
  const bool dma_v = grp == 1;
  const uint16_t* dsrc = (dma_v ? V : K) + head_kv;
  const uint32_t rs2 = (uint32_t)(rs_kv * 2);
  uint32_t doff[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = 16 * wl + 4 * r + (lane >> 4), p = lane & 15;
    const int c = dma_v ? (p ^ (2 * (row & 7))) : (p ^ (row & 15));
    doff[r] = (uint32_t)row * rs2 + 16u * (uint32_t)c;
  }
  uint8_t* const dlds = smem + (dma_v ? PP_VRING : 0) + wl * 4096;
  auto issue = [&](int tile, int slot) TLM_INLINE {
    const int valid = min(PP_KV, Sk - PP_KV * tile);
    const uint32_t nrec = (uint32_t)(valid - 1) * rs2 + PP_D * 2;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(dsrc + (int64_t)tile * PP_KV * rs_kv), (short)0, (int)nrec, PP_RSRC_WORD3);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc, (__attribute__((address_space(3))) void*)(dlds + slot * PP_TILE + r * 1024), 16,
          doff[r], 0, 0, NT ? CP_NT : PP_KV_CP);
  };

  // ---- operand read addresses (LDS byte addresses of the current K / V stage; row-block offsets
  // within a stage are immediates)
  const uint32_t sbase = lds_u32(smem);
  // K (A of S^T): key row 16 kt + ql (kt as an immediate row offset), d chunk 4 dk + g
  uint32_t kaddr[PP_D / 32];
#pragma unroll
  for (int dk = 0; dk < PP_D / 32; ++dk)
    kaddr[dk] = sbase + (uint32_t)(ql * 256 + 16 * ((4 * dk + g) ^ ql));
  // V^T (A of O^T) through ds_read_b64_tr_b16: 16-lane group g, lane j reads 4 dims
  // 16 dt + 4 (j % 4) of key row 4 g + j / 4 (+ 16 for the second read, + 32 for the second
  // k-step) and receives dim 16 dt + j of the four keys. The operand's k (key) set of lane
  // group g is {4 g .. 4 g + 3, 16 + 4 g .. 16 + 4 g + 3} of the 32-key step, the set in which
  // the S^T accumulators hold P^T (any key order gives the same product when P^T uses it too).
  const int jj = lane & 15;
  const int vrow = 4 * g + (jj >> 2);
  uint32_t vaddr[PP_D / 16];
#pragma unroll
  for (int dt = 0; dt < PP_D / 16; ++dt) {
    const int c = (2 * dt + ((jj & 3) >> 1)) ^ (2 * (vrow & 7));
    vaddr[dt] = sbase + PP_VRING + (uint32_t)(vrow * 256 + 16 * c + 8 * (jj & 1));
  }

  f32x4 oacc[PP_D / 16][2];  // O^T: [16-dim tile][query tile], element i = dim 16 dt + 4 g + i
#pragma unroll
  for (int t = 0; t < PP_D / 16; ++t) oacc[t][0] = oacc[t][1] = f32x4{};
  f32x4 sacc[4][2];  // S^T: [16-key tile][query tile], element i = key 16 kt + 4 g + i
  u32x4 pb[2][2];    // P^T operands of the last softmax: [32-key step][query tile]
  float m_run[2] = {-INFINITY, -INFINITY}, l_part[2] = {0.f, 0.f};

  // ---- MFMA phase: QK of the tile in the current K stage (16 operands x 2 query tiles), then
  // PV of the tile in the current V stage (16 operands x 2 query tiles). Operand reads run DEPTH
  // operands ahead.
  constexpr int DEPTH = 4;
  auto x_phase = [&](auto QKc, auto PVc) TLM_INLINE {
    constexpr bool DO_QK = decltype(QKc)::value, DO_PV = decltype(PVc)::value;
    constexpr int NQK = DO_QK ? 16 : 0;
    constexpr int NOPS = NQK + (DO_PV ? 16 : 0);
    u32x4 op[DEPTH + 1];
    auto read = [&](auto Mc) TLM_INLINE {
      constexpr int m = decltype(Mc)::value;
      if constexpr (m < NOPS) {
        if constexpr (m < NQK) {  // K rows 16 kt .. 16 kt + 15, d chunk 4 dk + g
          constexpr int dk = m / 4, kt = m % 4;
          op[m % (DEPTH + 1)] = ds_b128<kt * 16 * 256>(kaddr[dk]);
        } else {  // V^T: keys 32 ks + {4 g.., 16 + 4 g..}, dims 16 dt + ..
          constexpr int mm = m - NQK, ks = mm / 8, dt = mm % 8;
          constexpr int off = 32 * ks * 256;
          const u32x2 lo = ds_tr16<off>(vaddr[dt]);
          const u32x2 hi = ds_tr16<off + 16 * 256>(vaddr[dt]);
          op[m % (DEPTH + 1)] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
      }
    };
    constexpr auto nreads = [](int m) { return m < NQK ? 1 : 2; };
    __builtin_amdgcn_s_setprio(1);
    static_for<DEPTH>([&](auto Mc) TLM_INLINE { read(Mc); });
    static_for<NOPS>([&](auto Mc) TLM_INLINE {
      constexpr int m = decltype(Mc)::value;
      read(std::integral_constant<int, m + DEPTH>{});
      constexpr int pending = [&] {
        int c = 0;
        for (int i = m + 1; i <= m + DEPTH && i < NOPS; ++i) c += nreads(i);
        return c;
      }();
      lgkm_wait<pending>();
      order_after(op[m % (DEPTH + 1)]);
      const v8 a = __builtin_bit_cast(v8, op[m % (DEPTH + 1)]);
      if constexpr (m < NQK) {
        constexpr int dk = m / 4, kt = m % 4;
#pragma unroll
        for (int qq = 0; qq < 2; ++qq)
          sacc[kt][qq] = MT::mma(a, qreg[qq][dk], dk == 0 ? f32x4{} : sacc[kt][qq]);
      } else {
        constexpr int mm = m - NQK, ks = mm / 8, dt = mm % 8;
#pragma unroll
        for (int qq = 0; qq < 2; ++qq)
          oacc[dt][qq] = MT::mma(a, __builtin_bit_cast(v8, pb[ks][qq]), oacc[dt][qq]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    __builtin_amdgcn_s_setprio(0);
  };

  // ---- softmax of tile j (scores in sacc): lane holds keys 64 j + 16 kt + 4 g + i of queries
  // my_q[qq]. P = 2^(s sc - m) with the current m; the tile's P sum bounds every P, so a sum
  // above P_LIMIT (or not finite) sends the tile through the rescaling path. P_LIMIT keeps P in
  // range of the 16-bit type (fp16: every P <= 2^15) and O, l far from fp32 overflow (bf16:
  // P <= 2^64).
  constexpr float P_LIMIT = BF16 ? 18446744073709551616.0f : 32768.0f;
  auto exp_tile = [&](int qq, float nb) TLM_INLINE {  // fills pb[.][qq], returns the row-sum part
    float ts0 = 0.f, ts1 = 0.f;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float p0 = fast_exp2(__builtin_fmaf(sacc[kt][qq][2 * e], sc, nb));
        const float p1 = fast_exp2(__builtin_fmaf(sacc[kt][qq][2 * e + 1], sc, nb));
        if (e & 1) ts1 += p0 + p1; else ts0 += p0 + p1;
        pb[kt >> 1][qq][2 * (kt & 1) + e] = HH::pack(p0, p1);
      }
    return ts0 + ts1;
  };
  auto y_phase = [&](int j) TLM_INLINE {
    const int k0 = PP_KV * j;
    const bool need_mask = (CAUSAL && k0 + PP_KV - 1 > qb0 + coff) || (k0 + PP_KV > Sk);
    if (need_mask) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = k0 + 16 * kt + 4 * g + i;
#pragma unroll
          for (int qq = 0; qq < 2; ++qq)
            if (key >= Sk || (CAUSAL && key > my_q[qq] + coff)) sacc[kt][qq][i] = -INFINITY;
        }
    }
    // the first tile (m = -inf) always needs its max: skip the exponentials it would redo
    float ts[2] = {0.f, 0.f};
    if (j > 0) {
      ts[0] = exp_tile(0, -m_run[0]);
      ts[1] = exp_tile(1, -m_run[1]);
    }
    if (j == 0 || __builtin_amdgcn_ballot_w64(!(ts[0] <= P_LIMIT) || !(ts[1] <= P_LIMIT))) {
#pragma unroll
      for (int qq = 0; qq < 2; ++qq) {
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sacc[kt][qq][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run[qq], mx * sc);
        const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run[qq] - m_new);
        m_run[qq] = m_new;
        l_part[qq] *= alpha;
#pragma unroll
        for (int dt = 0; dt < PP_D / 16; ++dt) oacc[dt][qq] *= alpha;
        ts[qq] = exp_tile(qq, m_new == -INFINITY ? 0.f : -m_new);
      }
    }
    l_part[0] += ts[0];
    l_part[1] += ts[1];
  };

  // ---- schedule. Step j: group 0 runs X(j) = QK(j) + PV(j-1), then Y(j) = softmax(j); group 1
  // runs Y(j-1), then X(j). Both issue their half of tile j + 2 at the start of their Y half.
  // Tile j lives in stage j % 4: its K stage is read in step j and its V stage in step j + 1, so
  // the stage of tile j + 2 (that of tile j - 2) is free in step j. A wave runs the full X phase
  // in every step 1 .. nw: in step nw its QK reads a stage that holds finished data and the scores
  // are not used. Step 0 (no PV yet) is peeled.
  using T_ = std::true_type;
  using F_ = std::false_type;
  if (n > 0) issue(0, 0);
  if (n > 1) issue(1, 1);
  if (n > 1)
    vm_wait<4>();
  else
    vm_wait<0>();
  phase_barrier();
  // stage offsets of step j: K stage j % 4, V stage (j - 1) % 4
  auto advance = [&](int j) TLM_INLINE {
    const int dk = (j & 3) == 0 ? -3 * PP_TILE : PP_TILE;
#pragma unroll
    for (int d = 0; d < PP_D / 32; ++d) kaddr[d] += dk;
    if (j >= 2) {
      const int dv = ((j - 1) & 3) == 0 ? -3 * PP_TILE : PP_TILE;
#pragma unroll
      for (int dt = 0; dt < PP_D / 16; ++dt) vaddr[dt] += dv;
    }
  };
  auto end_step = [&](bool dma) TLM_INLINE {
    if (dma)
      vm_wait<4>();
    else
      vm_wait<0>();
    phase_barrier();
  };
  if (n > 0) {
    if (grp == 0) {
      if (nw > 0) x_phase(T_{}, F_{});
      phase_barrier();
      if (2 < n) issue(2, 2);
      if (nw > 0) y_phase(0);
      end_step(2 < n);
      for (int j = 1; j <= n; ++j) {
        advance(j);
        if (j <= nw) x_phase(T_{}, T_{});
        phase_barrier();
        if (j + 2 < n) issue(j + 2, (j + 2) & 3);
        if (j < nw) y_phase(j);
        end_step(j + 2 < n);
      }
    } else {
      if (2 < n) issue(2, 2);
      phase_barrier();
      if (nw > 0) x_phase(T_{}, F_{});
      end_step(2 < n);
      for (int j = 1; j <= n; ++j) {
        advance(j);
        if (j + 2 < n) issue(j + 2, (j + 2) & 3);
        if (j <= nw) y_phase(j - 1);
        phase_barrier();
        if (j <= nw) x_phase(T_{}, T_{});
        end_step(j + 2 < n);
      }
    }
  }

  // ---- epilogue: lane holds O^T[d = 16 dt + 4 g + i][query my_q[qq]]; the row sums of a query
  // are spread over the four lane groups
  float inv[2], l_all[2];
#pragma unroll
  for (int qq = 0; qq < 2; ++qq) {
    float l_tot = l_part[qq] + __shfl_xor(l_part[qq], 16, 64);
    l_tot += __shfl_xor(l_tot, 32, 64);
    l_all[qq] = l_tot;
    inv[qq] = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  }
  if constexpr (OUT32) {  // fp32 output (fp32 programs, split parts): 16-byte stores from registers
    int64_t ob = head, ors = rs;
    if constexpr (SPLIT) {  // part si of query q: row ((b S_q + q) H + h) nsi + si
      ob = ((sr.q0 * H + h) * sp.nsi + si) * PP_D;
      ors = (int64_t)H * sp.nsi * PP_D;
    }
    float* Of = (float*)O + ob;
#pragma unroll
    for (int qq = 0; qq < 2; ++qq)
      if (my_q[qq] < Sq) {
#pragma unroll
        for (int dt = 0; dt < PP_D / 16; ++dt)
          *(f32x4*)(Of + (int64_t)my_q[qq] * ors + 16 * dt + 4 * g) = oacc[dt][qq] * inv[qq];
        if constexpr (SPLIT) {
          if (g == 0)
            sp.lse[ob / PP_D + (int64_t)my_q[qq] * ors / PP_D] =
                l_all[qq] > 0.f ? m_run[qq] + __log2f(l_all[qq]) : -INFINITY;
        }
      }
    return;
  }
  uint16_t* stage = (uint16_t*)smem + wave * 32 * PP_OP;  // [32 queries][PP_OP]
#pragma unroll
  for (int qq = 0; qq < 2; ++qq)
#pragma unroll
    for (int dt = 0; dt < PP_D / 16; ++dt) {
      const f32x4 o = oacc[dt][qq] * inv[qq];
      *(u32x2*)(stage + (16 * qq + ql) * PP_OP + 16 * dt + 4 * g) =
          u32x2{HH::pack(o[0], o[1]), HH::pack(o[2], o[3])};
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  uint16_t* Ob = (uint16_t*)O + head;
#pragma unroll
  for (int it = 0; it < 32 * (PP_D / 8) / 64; ++it) {
    const int idx = lane + 64 * it;
    const int r = idx / (PP_D / 8), c = (idx % (PP_D / 8)) * 8;
    const int q = qb0 + r;
    if (q < Sq) *(u32x4*)(Ob + (int64_t)q * rs + c) = *(const u32x4*)(stage + r * PP_OP + c);
  }
  }();
  // the next tile's LDS-DMA overwrites the epilogue's staging: every wave has read its own
  phase_barrier();
  }
}

template <bool BF16, bool CAUSAL, bool OUT32, bool SPLIT = false, bool NT = false>
int launch_pp(const void* q, const void* k, const void* v, void* o, int B, int S, int H, int Hkv,
              float sc, const SeqMap& sm, hipStream_t st, const FaSplit& sp = FaSplit{}) {
  const int64_t nqt = (S + PP_BQ - 1) / PP_BQ;
  // causal: two tiles per workgroup; split: one workgroup per internal key split
  const int64_t nwg = (CAUSAL ? (nqt + 1) / 2 : nqt) * B * H * (SPLIT ? sp.nsi : 1);
  if (nwg > INT32_MAX) {
    tlm_set_error("tlm_flash_attn_fwd: problem too large");
    return TLM_EINVAL;
  }
  fa_fwd_pp<BF16, CAUSAL, OUT32, SPLIT, NT><<<(unsigned)nwg, 512, 0, st>>>(
      (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, o, B, S, H, Hkv, sc, sm, sp);
  TLM_LAUNCH_CHECK("tlm_flash_attn_fwd");
  return TLM_OK;
}

template <bool BF16, bool CAUSAL, int D>
int launch(const void* q, const void* k, const void* v, void* o, int B, int S, int H, int Hkv,
           float sc, const SeqMap& sm, hipStream_t st) {
  const int64_t nwg = (int64_t)((S + BQ - 1) / BQ) * B * H;
  if (nwg > INT32_MAX) {
    tlm_set_error("tlm_flash_attn_fwd: problem too large");
    return TLM_EINVAL;
  }
  fa_fwd<BF16, CAUSAL, D><<<(unsigned)nwg, 64 * FA_WAVES, 0, st>>>(
      (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, B, S, H, Hkv, sc,
      sm);
  TLM_LAUNCH_CHECK("tlm_flash_attn_fwd");
  return TLM_OK;
}

// ---- any head dim (multiple of 8, <= 256): the demo programs' own shapes (dim 8) and head dims
// without a tiled kernel. One query per lane with q and O in registers; key and value rows are
// read with wave-uniform addresses; per key the online softmax of the reference (m = running
// max, alpha = 2^(m_prev - m), P = 2^(s sc - m) rounded to the input type before P V, l from
// the fp32 P). No MFMA: for shapes far too small to fill matrix tiles.
template <bool BF16, bool CAUSAL, bool OUT32, int DC,  // DC = capacity in 8-element chunks
          bool SPLIT = false>
__global__ __launch_bounds__(256) void fa_fwd_generic(const uint16_t* __restrict__ Q,
                                                      const uint16_t* __restrict__ K,
                                                      const uint16_t* __restrict__ V,
                                                      void* __restrict__ O, int H, int Hkv,
                                                      int D, float sc, SeqMap sm, FaSplit sp) {
  static_assert(!SPLIT || (OUT32 && !CAUSAL), "split parts are non-causal with fp32 output");
  using HH = h16<BF16>;
  const int si = SPLIT ? (int)(blockIdx.y % sp.nsi) : 0;
  const int bh = SPLIT ? (int)(blockIdx.y / sp.nsi) : (int)blockIdx.y, b = bh / H, h = bh % H;
  SeqRange sr = seq_range(sm, b);
  if constexpr (SPLIT) sr = split_keys(sr, sp, si);
  const int S = sr.nq, Sk = sr.nk, coff = Sk - S;  // causal: query i sees keys j <= i + coff
  if ((int)blockIdx.x * 256 >= S) return;  // whole block
  const int q = blockIdx.x * 256 + threadIdx.x;
  const int nc = D / 8;
  const int64_t rs = sm.tq, rs_kv = sm.tk;
  const int64_t head = sr.q0 * H * D + h * sm.hq;
  const int64_t head_kv = sr.k0 * Hkv * D + (h / (H / Hkv)) * sm.hk;
  u32x4 qv[DC];
  float o[DC][8];
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    qv[c] = u32x4{0, 0, 0, 0};
    if (c < nc && q < S) qv[c] = *(const u32x4*)(Q + head + (int64_t)q * rs + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[c][e] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  // keys of the wave: causal stops after the wave's last query (wave-uniform bound)
  const int wq_last = min(S - 1, (int)(blockIdx.x * 256 + (threadIdx.x & ~63) + 63));
  const int kend = CAUSAL ? max(0, min(Sk, wq_last + coff + 1)) : Sk;
  for (int j = 0; j < kend; ++j) {
    const uint16_t* kr = K + head_kv + (int64_t)j * rs_kv;
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      if (c < nc) {
        const u32x4 kc = *(const u32x4*)(kr + 8 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s = fmaf(HH::lo(qv[c][e]), HH::lo(kc[e]), s);
          s = fmaf(HH::hi(qv[c][e]), HH::hi(kc[e]), s);
        }
      }
    }
    s *= sc;
    if (CAUSAL && j > q + coff) s = -INFINITY;
    const float m_new = fmaxf(m, s);
    const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m - m_new);
    const float p = m_new == -INFINITY ? 0.f : fast_exp2(s - m_new);
    const float pr = HH::to_f32(HH::from_f32(p));
    l = fmaf(l, alpha, p);
    m = m_new;
    const uint16_t* vr = V + head_kv + (int64_t)j * rs_kv;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      if (c < nc) {
        const u32x4 vc = *(const u32x4*)(vr + 8 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[c][2 * e] = fmaf(o[c][2 * e], alpha, pr * HH::lo(vc[e]));
          o[c][2 * e + 1] = fmaf(o[c][2 * e + 1], alpha, pr * HH::hi(vc[e]));
        }
      }
    }
  }
  if (q >= S) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  int64_t ob = head, ors = rs;
  if constexpr (SPLIT) {  // part si of query q: row ((b S_q + q) H + h) nsi + si
    ob = ((sr.q0 * H + h) * sp.nsi + si) * D;
    ors = (int64_t)H * sp.nsi * D;
    sp.lse[ob / D + (int64_t)q * ors / D] = l > 0.f ? m + __log2f(l) : -INFINITY;
  }
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    if (c < nc) {
      const int64_t off = ob + (int64_t)q * ors + 8 * c;
      if constexpr (OUT32) {
        float* Of = (float*)O + off;
        *(f32x4*)Of = f32x4{o[c][0] * inv, o[c][1] * inv, o[c][2] * inv, o[c][3] * inv};
        *(f32x4*)(Of + 4) = f32x4{o[c][4] * inv, o[c][5] * inv, o[c][6] * inv, o[c][7] * inv};
      } else {
        *(u32x4*)((uint16_t*)O + off) =
            u32x4{HH::pack(o[c][0] * inv, o[c][1] * inv), HH::pack(o[c][2] * inv, o[c][3] * inv),
                  HH::pack(o[c][4] * inv, o[c][5] * inv), HH::pack(o[c][6] * inv, o[c][7] * inv)};
      }
    }
  }
}

// All-fp32 attention (tpu_demo/ppl/flashattn/fa_fp32.py: fp32 Q, K, V, fp32 score and P tiles,
// fp32 output): the generic per-query kernel with fp32 operands and no rounding of P. One query
// per lane, q and O in VGPRs (DC chunks of 4 floats), keys read with wave-uniform addresses.
template <bool CAUSAL, int DC>  // DC = capacity in 4-element chunks
__global__ __launch_bounds__(256) void fa_fwd_generic_f32(const float* __restrict__ Q,
                                                          const float* __restrict__ K,
                                                          const float* __restrict__ V,
                                                          float* __restrict__ O, int H, int Hkv,
                                                          int D, float sc, SeqMap sm) {
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const SeqRange sr = seq_range(sm, b);
  const int S = sr.nq, Sk = sr.nk, coff = Sk - S;
  if ((int)blockIdx.x * 256 >= S) return;
  const int q = blockIdx.x * 256 + threadIdx.x;
  const int nc = D / 4;
  const int64_t rs = sm.tq, rs_kv = sm.tk;
  const int64_t head = sr.q0 * H * D + h * sm.hq;
  const int64_t head_kv = sr.k0 * Hkv * D + (h / (H / Hkv)) * sm.hk;
  f32x4 qv[DC], o[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    qv[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    o[c] = qv[c];
    if (c < nc && q < S) qv[c] = *(const f32x4*)(Q + head + (int64_t)q * rs + 4 * c);
  }
  float m = -INFINITY, l = 0.f;
  const int wq_last = min(S - 1, (int)(blockIdx.x * 256 + (threadIdx.x & ~63) + 63));
  const int kend = CAUSAL ? max(0, min(Sk, wq_last + coff + 1)) : Sk;
  for (int j = 0; j < kend; ++j) {
    const float* kr = K + head_kv + (int64_t)j * rs_kv;
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      if (c < nc) {
        const f32x4 kc = *(const f32x4*)(kr + 4 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) s = fmaf(qv[c][e], kc[e], s);
      }
    }
    s *= sc;
    if (CAUSAL && j > q + coff) s = -INFINITY;
    const float m_new = fmaxf(m, s);
    const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m - m_new);
    const float p = m_new == -INFINITY ? 0.f : fast_exp2(s - m_new);
    l = fmaf(l, alpha, p);
    m = m_new;
    const float* vr = V + head_kv + (int64_t)j * rs_kv;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      if (c < nc) {
        const f32x4 vc = *(const f32x4*)(vr + 4 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[c][e] = fmaf(o[c][e], alpha, p * vc[e]);
      }
    }
  }
  if (q >= S) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
  for (int c = 0; c < DC; ++c)
    if (c < nc) *(f32x4*)(O + head + (int64_t)q * rs + 4 * c) = o[c] * inv;
}

template <bool CAUSAL>
int launch_generic_f32(const void* q, const void* k, const void* v, void* o, int B, int S, int H,
                       int Hkv, int D, float sc, const SeqMap& sm, hipStream_t st) {
  if ((int64_t)B * H > 65535) {
    tlm_set_error("tlm_flash_attn_fwd: fp32 attention needs batch * heads <= 65535");
    return TLM_EUNSUPPORTED;
  }
  const dim3 grid((unsigned)((S + 255) / 256), (unsigned)(B * H));
  auto go = [&](auto kern) {
    kern<<<grid, 256, 0, st>>>((const float*)q, (const float*)k, (const float*)v, (float*)o, H,
                               Hkv, D, sc, sm);
  };
  if (D <= 16)
    go(fa_fwd_generic_f32<CAUSAL, 4>);
  else if (D <= 64)
    go(fa_fwd_generic_f32<CAUSAL, 16>);
  else if (D <= 128)
    go(fa_fwd_generic_f32<CAUSAL, 32>);
  else
    go(fa_fwd_generic_f32<CAUSAL, 64>);
  TLM_LAUNCH_CHECK("tlm_flash_attn_fwd (fp32)");
  return TLM_OK;
}

template <bool BF16, bool CAUSAL, bool OUT32, bool SPLIT = false>
int launch_generic(const void* q, const void* k, const void* v, void* o, int B, int S, int H,
                   int Hkv, int D, float sc, const SeqMap& sm, hipStream_t st,
                   const FaSplit& sp = FaSplit{}) {
  const int64_t ny = (int64_t)B * H * (SPLIT ? sp.nsi : 1);
  if (ny > 65535) {
    tlm_set_error("tlm_flash_attn_fwd: head dim %d needs batch * heads%s <= 65535", D,
                  SPLIT ? " * key parts" : "");
    return TLM_EUNSUPPORTED;
  }
  const dim3 grid((unsigned)((S + 255) / 256), (unsigned)ny);
  auto go = [&](auto kern) {
    kern<<<grid, 256, 0, st>>>((const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, o, H,
                               Hkv, D, sc, sm, sp);
  };
  if (D <= 16)
    go(fa_fwd_generic<BF16, CAUSAL, OUT32, 2, SPLIT>);
  else if (D <= 64)
    go(fa_fwd_generic<BF16, CAUSAL, OUT32, 8, SPLIT>);
  else if (D <= 128)
    go(fa_fwd_generic<BF16, CAUSAL, OUT32, 16, SPLIT>);
  else
    go(fa_fwd_generic<BF16, CAUSAL, OUT32, 32, SPLIT>);
  TLM_LAUNCH_CHECK("tlm_flash_attn_fwd");
  return TLM_OK;
}

// Combine of the split-KV inference program (example_mha_inference.py:162-203, reduce_ref
// :216-227). Thread = (row = (b, q, h), 4 dims). Each program split s first merges its r internal
// parts exactly (fp32), and its result is stored as the program's partial in the 16-bit dtype:
// Output_partial[b, q, h, s, :] = O_s and glse[b, h, s, q] = lse_s (log2 domain). Output is then
// the merge of those stored (rounded) values, as the program's combine reads them back:
// O = sum_s O_s 2^(lse_s - lse), lse = log2 sum_s 2^(lse_s) (taken here as a running merge).
constexpr int FA_MAX_PARTS = 8;  // internal parts per program split
// RA > 0: every part of every split (r == RA, ns RA <= FA_ALL_PARTS) is requested before any is
// used, so a thread waits for one memory latency instead of one per split; RA == 0: any r, one
// split's parts at a time.
constexpr int FA_ALL_PARTS = 16;
template <bool BF16, int RA>
__global__ __launch_bounds__(256) void fa_split_combine(const float* __restrict__ part,
                                                        const float* __restrict__ lse,
                                                        uint16_t* __restrict__ glse,
                                                        uint16_t* __restrict__ opart,
                                                        uint16_t* __restrict__ out, int64_t rows,
                                                        int Sq, int H, int D, int ns, int r) {
  using HH = h16<BF16>;
  const int nch = D / 4;
  const int64_t gt = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gt / nch;
  if (row >= rows) return;
  const int c = (int)(gt % nch);
  const int h = (int)(row % H);
  const int64_t bq = row / H;
  const int q = (int)(bq % Sq);
  const int64_t b = bq / Sq;
  const int nsi = ns * r;
  float M = -INFINITY, L = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // split sp from its parts (lse lv, output pv; absent parts have lse -inf and weigh 0)
  auto merge_split = [&](int sp, const float* lv, const f32x4* pv, int np) {
    float m = -INFINITY;
    for (int j = 0; j < np; ++j) m = fmaxf(m, lv[j]);
    float l = 0.f;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    if (m != -INFINITY) {
      for (int j = 0; j < np; ++j) {
        const float w = fast_exp2(lv[j] - m);  // 0 for an empty or absent part
        l += w;
        o += pv[j] * w;
      }
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    const u32x2 pk = u32x2{HH::pack(o[0] * inv, o[1] * inv), HH::pack(o[2] * inv, o[3] * inv)};
    *(u32x2*)(opart + (row * ns + sp) * D + 4 * c) = pk;
    const uint32_t lb = HH::from_f32(l > 0.f ? m + __log2f(l) : -INFINITY);
    if (c == 0) glse[((b * H + h) * ns + sp) * Sq + q] = (uint16_t)lb;
    // merge the stored values, as read back: running max and sum of 2^lse
    const float lr = HH::to_f32(lb);
    if (lr != -INFINITY) {
      const float Mn = fmaxf(M, lr);
      const float a = fast_exp2(M - Mn), w = fast_exp2(lr - Mn);  // a = 0 while M = -inf
      L = L * a + w;
      acc = acc * a + f32x4{HH::lo(pk[0]), HH::hi(pk[0]), HH::lo(pk[1]), HH::hi(pk[1])} * w;
      M = Mn;
    }
  };
  if constexpr (RA > 0) {
    float la[FA_ALL_PARTS];
    f32x4 pa[FA_ALL_PARTS];
#pragma unroll
    for (int k = 0; k < FA_ALL_PARTS; ++k) {
      la[k] = -INFINITY;
      pa[k] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (k < nsi) {
        la[k] = lse[row * nsi + k];
        pa[k] = *(const f32x4*)(part + (row * nsi + k) * D + 4 * c);
      }
    }
#pragma unroll
    for (int sp = 0; sp < FA_ALL_PARTS / RA; ++sp)
      if (sp < ns) merge_split(sp, la + sp * RA, pa + sp * RA, RA);
  } else {
    for (int sp = 0; sp < ns; ++sp) {
      // every part of the split requested before any is used
      float lv[FA_MAX_PARTS];
      f32x4 pv[FA_MAX_PARTS];
#pragma unroll
      for (int j = 0; j < FA_MAX_PARTS; ++j) {
        lv[j] = -INFINITY;
        pv[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (j < r) {
          const int64_t pi = row * nsi + sp * r + j;
          lv[j] = lse[pi];
          pv[j] = *(const f32x4*)(part + pi * D + 4 * c);
        }
      }
      merge_split(sp, lv, pv, FA_MAX_PARTS);
    }
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  *(u32x2*)(out + row * D + 4 * c) =
      u32x2{HH::pack(acc[0] * inv, acc[1] * inv), HH::pack(acc[2] * inv, acc[3] * inv)};
}

// Internal key parts per program split: enough workgroups for every CU, each part at least
// eight 64-key tiles. Shared by the launch and the workspace query.
int split_parts(int64_t B, int64_t S_q, int64_t S_kv, int64_t H, int64_t D, int ns) {
  const int64_t per = S_kv / ns;
  const int64_t qtiles = D == 128 ? (S_q + PP_BQ - 1) / PP_BQ : (S_q + 255) / 256;
  const int64_t base = std::max<int64_t>(1, B * H * qtiles * ns);
  int64_t r = (256 + base - 1) / base;
  r = std::min<int64_t>(r, std::max<int64_t>(1, per / (8 * PP_KV)));
  return (int)std::max<int64_t>(1, std::min<int64_t>(r, FA_MAX_PARTS));
}

// S: queries per sequence (dense) or the longest sequence's (variable length); sm: row ranges.
template <bool BF16, bool OUT32>
int by_shape(const void* q, const void* k, const void* v, void* o, int B, int S, int H, int Hkv,
             int D, bool causal, float sc, const SeqMap& sm, hipStream_t st) {
  if (D == 128)
    return causal ? launch_pp<BF16, true, OUT32>(q, k, v, o, B, S, H, Hkv, sc, sm, st)
                  : launch_pp<BF16, false, OUT32>(q, k, v, o, B, S, H, Hkv, sc, sm, st);
  if (D == 64 && !OUT32)
    return causal ? launch<BF16, true, 64>(q, k, v, o, B, S, H, Hkv, sc, sm, st)
                  : launch<BF16, false, 64>(q, k, v, o, B, S, H, Hkv, sc, sm, st);
  return causal ? launch_generic<BF16, true, OUT32>(q, k, v, o, B, S, H, Hkv, D, sc, sm, st)
                : launch_generic<BF16, false, OUT32>(q, k, v, o, B, S, H, Hkv, D, sc, sm, st);
}

// Checks shared by the dense and variable-length entry points.
int check_common(const char* fn, const void* q, const void* k, const void* v, const void* o,
                 int64_t H, int64_t H_kv, int64_t D, float sm_scale, int in_dtype,
                 int out_dtype) {
  if (!q || !k || !v || !o) {
    tlm_set_error("%s: null pointer argument", fn);
    return TLM_EINVAL;
  }
  if (H < 0 || H > 65535) {
    tlm_set_error("%s: bad head count %lld", fn, (long long)H);
    return TLM_EINVAL;
  }
  if (H_kv <= 0 || H_kv > H || H % H_kv != 0) {
    tlm_set_error("%s: %lld query heads do not split into groups of %lld K/V heads", fn,
                  (long long)H, (long long)H_kv);
    return TLM_EINVAL;
  }
  if (D <= 0 || D > 256 || D % (in_dtype == TLM_F32 ? 4 : 8) != 0) {
    tlm_set_error("%s: head dim %lld unsupported (a multiple of 8, or of 4 for fp32, at most "
                  "256)", fn, (long long)D);
    return TLM_EUNSUPPORTED;
  }
  if (in_dtype != TLM_BF16 && in_dtype != TLM_F16 && in_dtype != TLM_F32) {
    tlm_set_error("%s: dtype %d unsupported (BF16, F16 or F32)", fn, in_dtype);
    return TLM_EUNSUPPORTED;
  }
  if (out_dtype != in_dtype && out_dtype != TLM_F32) {
    tlm_set_error("%s: output dtype %d unsupported (the input dtype or F32)", fn, out_dtype);
    return TLM_EUNSUPPORTED;
  }
  if (!(sm_scale > 0.f) || !__builtin_isfinite(sm_scale)) {
    tlm_set_error("%s: sm_scale must be positive and finite", fn);
    return TLM_EINVAL;
  }
  if (!tlm_aligned(q, 16) || !tlm_aligned(k, 16) || !tlm_aligned(v, 16) || !tlm_aligned(o, 16)) {
    tlm_set_error("%s: tensors must be 16-byte aligned", fn);
    return TLM_EINVAL;
  }
  return TLM_OK;
}

int dispatch(const void* q, const void* k, const void* v, void* o, int B, int S, int H, int Hkv,
             int D, bool causal, float sm_scale, int in_dtype, int out_dtype, const SeqMap& sm,
             hipStream_t st) {
  const float sc = (float)((double)sm_scale * 1.4426950408889634);
  if (in_dtype == TLM_F32)
    return causal ? launch_generic_f32<true>(q, k, v, o, B, S, H, Hkv, D, sc, sm, st)
                  : launch_generic_f32<false>(q, k, v, o, B, S, H, Hkv, D, sc, sm, st);
  const bool bf = in_dtype == TLM_BF16, f32o = out_dtype == TLM_F32;
  if (bf)
    return f32o ? by_shape<true, true>(q, k, v, o, B, S, H, Hkv, D, causal, sc, sm, st)
                : by_shape<true, false>(q, k, v, o, B, S, H, Hkv, D, causal, sc, sm, st);
  return f32o ? by_shape<false, true>(q, k, v, o, B, S, H, Hkv, D, causal, sc, sm, st)
              : by_shape<false, false>(q, k, v, o, B, S, H, Hkv, D, causal, sc, sm, st);
}

}  // namespace

extern "C" int tlm_flash_attn_fwd_ex(const void* q, const void* k, const void* v, void* o,
                                     int64_t B, int64_t S, int64_t H, int64_t H_kv, int64_t D,
                                     int causal, float sm_scale, int in_dtype, int out_dtype,
                                     void* stream) {
  const int rc = check_common("tlm_flash_attn_fwd", q, k, v, o, H, H_kv, D, sm_scale, in_dtype,
                              out_dtype);
  if (rc != TLM_OK) return rc;
  if (B < 0 || S < 0 || B > 65535 || S > (1 << 24)) {
    tlm_set_error("tlm_flash_attn_fwd: bad shape");
    return TLM_EINVAL;
  }
  if (B == 0 || S == 0 || H == 0) return TLM_OK;
  const SeqMap sm{nullptr, nullptr, (int)S, (int)S, H * D, H_kv * D, D, D};
  return dispatch(q, k, v, o, (int)B, (int)S, (int)H, (int)H_kv, (int)D, causal != 0, sm_scale,
                  in_dtype, out_dtype, sm, (hipStream_t)stream);
}

extern "C" int tlm_flash_attn_varlen_fwd(const void* q, const void* k, const void* v, void* o,
                                         const int32_t* cu_seqlens_q,
                                         const int32_t* cu_seqlens_k, int64_t B,
                                         int64_t max_seqlen_q, int64_t total_q, int64_t total_k,
                                         int64_t H, int64_t H_kv, int64_t D, int causal,
                                         float sm_scale, int in_dtype, int out_dtype,
                                         void* stream) {
  const int rc = check_common("tlm_flash_attn_varlen_fwd", q, k, v, o, H, H_kv, D, sm_scale,
                              in_dtype, out_dtype);
  if (rc != TLM_OK) return rc;
  if (!cu_seqlens_q || !cu_seqlens_k || !tlm_aligned(cu_seqlens_q, 4) ||
      !tlm_aligned(cu_seqlens_k, 4)) {
    tlm_set_error("tlm_flash_attn_varlen_fwd: cu_seqlens must be non-null, 4-byte aligned");
    return TLM_EINVAL;
  }
  if (B < 0 || B > 65535 || max_seqlen_q < 0 || max_seqlen_q > (1 << 24) || total_q < 0 ||
      total_k < 0 || total_q > INT32_MAX || total_k > INT32_MAX) {
    tlm_set_error("tlm_flash_attn_varlen_fwd: bad shape");
    return TLM_EINVAL;
  }
  if (B == 0 || max_seqlen_q == 0 || H == 0 || total_q == 0) return TLM_OK;
  const SeqMap sm{cu_seqlens_q, cu_seqlens_k, (int)total_q, (int)total_k, H * D, H_kv * D, D, D};
  return dispatch(q, k, v, o, (int)B, (int)max_seqlen_q, (int)H, (int)H_kv, (int)D, causal != 0,
                  sm_scale, in_dtype, out_dtype, sm, (hipStream_t)stream);
}

extern "C" int tlm_flash_attn_bhsd_fwd(const void* q, const void* k, const void* v, void* o,
                                       int64_t B, int64_t H, int64_t H_kv, int64_t S_q,
                                       int64_t S_kv, int64_t D, int causal, float sm_scale,
                                       int in_dtype, int out_dtype, void* stream) {
  const int rc = check_common("tlm_flash_attn_bhsd_fwd", q, k, v, o, H, H_kv, D, sm_scale,
                              in_dtype, out_dtype);
  if (rc != TLM_OK) return rc;
  if (B < 0 || S_q < 0 || S_kv < 0 || B > 65535 || S_q > (1 << 24) || S_kv > (1 << 24)) {
    tlm_set_error("tlm_flash_attn_bhsd_fwd: bad shape");
    return TLM_EINVAL;
  }
  if (B == 0 || S_q == 0 || H == 0) return TLM_OK;
  // query i sees keys j <= i + S_kv - S_q when causal (bottom-right diagonal); no keys: zero rows
  const SeqMap sm{nullptr, nullptr, (int)S_q, (int)S_kv, D, D, S_q * D, S_kv * D};
  return dispatch(q, k, v, o, (int)B, (int)S_q, (int)H, (int)H_kv, (int)D, causal != 0,
                  sm_scale, in_dtype, out_dtype, sm, (hipStream_t)stream);
}

extern "C" size_t tlm_flash_attn_splitkv_workspace_bytes(int64_t B, int64_t S_q, int64_t S_kv,
                                                         int64_t H, int64_t D, int num_split) {
  if (B <= 0 || S_q <= 0 || S_kv <= 0 || H <= 0 || D <= 0 || num_split <= 0 ||
      num_split > 16 || S_kv % num_split)
    return 0;
  const int r = split_parts(B, S_q, S_kv, H, D, num_split);
  return (size_t)B * S_q * H * num_split * r * (D + 1) * sizeof(float);
}

extern "C" int tlm_flash_attn_splitkv_fwd(const void* q, const void* k, const void* v, void* glse,
                                          void* o_partial, void* o, void* ws, size_t ws_bytes,
                                          int64_t B, int64_t S_q, int64_t S_kv, int64_t H,
                                          int64_t H_kv, int64_t D, int num_split, float sm_scale,
                                          int dtype, void* stream) {
  const char* fn = "tlm_flash_attn_splitkv_fwd";
  int rc = check_common(fn, q, k, v, o, H, H_kv, D, sm_scale, dtype, dtype);
  if (rc != TLM_OK) return rc;
  if (dtype == TLM_F32) {
    tlm_set_error("%s: dtype must be F16 or BF16", fn);
    return TLM_EUNSUPPORTED;
  }
  if (!glse || !o_partial || !ws || !tlm_aligned(glse, 2) || !tlm_aligned(o_partial, 16) ||
      !tlm_aligned(ws, 16)) {
    tlm_set_error("%s: glse, Output_partial and the workspace must be non-null and aligned (2, "
                  "16, 16 bytes)", fn);
    return TLM_EINVAL;
  }
  if (num_split < 1 || num_split > 16) {
    tlm_set_error("%s: num_split %d outside [1, 16]", fn, num_split);
    return TLM_EUNSUPPORTED;
  }
  if (B < 0 || S_q < 0 || S_kv < 0 || B > 65535 || S_q > (1 << 24) || S_kv > (1 << 24) ||
      S_kv % num_split) {
    tlm_set_error("%s: bad shape (S_kv must be a multiple of num_split)", fn);
    return TLM_EINVAL;
  }
  if (B == 0 || S_q == 0 || H == 0) return TLM_OK;
  if (S_kv == 0) {
    tlm_set_error("%s: no keys", fn);
    return TLM_EINVAL;
  }
  const size_t need = tlm_flash_attn_splitkv_workspace_bytes(B, S_q, S_kv, H, D, num_split);
  if (ws_bytes < need) {
    tlm_set_error("%s: workspace of %zu bytes, %zu needed", fn, ws_bytes, need);
    return TLM_EWORKSPACE;
  }
  const int r = split_parts(B, S_q, S_kv, H, D, num_split);
  const int per = (int)(S_kv / num_split);
  const int per_i = (per + r - 1) / r;
  const int64_t rows = B * S_q * H;
  float* part = (float*)ws;
  float* lse = part + rows * num_split * r * D;
  const bool once = (S_q + PP_BQ - 1) / PP_BQ == 1 && H_kv == H;  // each K / V tile read once
  const FaSplit sp{lse, num_split * r, r, per, per_i};
  const SeqMap sm{nullptr, nullptr, (int)S_q, (int)S_kv, H * D, H_kv * D, D, D};
  const float sc = (float)((double)sm_scale * 1.4426950408889634);
  hipStream_t st = (hipStream_t)stream;
  const bool bf = dtype == TLM_BF16;
  if (D == 128 && once)
    rc = bf ? launch_pp<true, false, true, true, true>(q, k, v, part, (int)B, (int)S_q, (int)H,
                                                       (int)H_kv, sc, sm, st, sp)
            : launch_pp<false, false, true, true, true>(q, k, v, part, (int)B, (int)S_q, (int)H,
                                                        (int)H_kv, sc, sm, st, sp);
  else if (D == 128)
    rc = bf ? launch_pp<true, false, true, true>(q, k, v, part, (int)B, (int)S_q, (int)H,
                                                 (int)H_kv, sc, sm, st, sp)
            : launch_pp<false, false, true, true>(q, k, v, part, (int)B, (int)S_q, (int)H,
                                                  (int)H_kv, sc, sm, st, sp);
  else
    rc = bf ? launch_generic<true, false, true, true>(q, k, v, part, (int)B, (int)S_q, (int)H,
                                                      (int)H_kv, (int)D, sc, sm, st, sp)
            : launch_generic<false, false, true, true>(q, k, v, part, (int)B, (int)S_q, (int)H,
                                                       (int)H_kv, (int)D, sc, sm, st, sp);
  if (rc != TLM_OK) return rc;
  const int64_t nthr = rows * (D / 4);
  const dim3 grid((unsigned)((nthr + 255) / 256));
  auto combine = [&](auto kern) {
    kern<<<grid, 256, 0, st>>>(part, lse, (uint16_t*)glse, (uint16_t*)o_partial, (uint16_t*)o,
                               rows, (int)S_q, (int)H, (int)D, num_split, r);
  };
  // all parts in one round when r is 1, 2, 4 or 8 and ns r <= FA_ALL_PARTS
  const bool all = num_split * r <= FA_ALL_PARTS && (r & (r - 1)) == 0;
  if (bf) {
    if (all && r == 1) combine(fa_split_combine<true, 1>);
    else if (all && r == 2) combine(fa_split_combine<true, 2>);
    else if (all && r == 4) combine(fa_split_combine<true, 4>);
    else if (all && r == 8) combine(fa_split_combine<true, 8>);
    else combine(fa_split_combine<true, 0>);
  } else {
    if (all && r == 1) combine(fa_split_combine<false, 1>);
    else if (all && r == 2) combine(fa_split_combine<false, 2>);
    else if (all && r == 4) combine(fa_split_combine<false, 4>);
    else if (all && r == 8) combine(fa_split_combine<false, 8>);
    else combine(fa_split_combine<false, 0>);
  }
  TLM_LAUNCH_CHECK("tlm_flash_attn_splitkv_fwd (combine)");
  return TLM_OK;
}

extern "C" int tlm_flash_attn_fwd(const void* q, const void* k, const void* v, void* o,
                                  int64_t B, int64_t S, int64_t H, int64_t D, int causal,
                                  float sm_scale, int dtype, void* stream) {
  return tlm_flash_attn_fwd_ex(q, k, v, o, B, S, H, H, D, causal, sm_scale, dtype, dtype, stream);
}
