// MLA paged decode (FP8 / fp16 / bf16 latent KV) and the paged-gather integer-path check.
//
// Reference: examples/deepseek_mla/example_mla_decode_paged.py
//   split kernel (:100-183): per (sequence, head block, split), loop over KV tiles of the split's
//     token range, page address kv_start = BT[b, tok / page] * page + tok % page (:147-148),
//     S = Q KV^T + Q_pe K_pe^T, tokens >= seqlen masked to -inf (:162-164), online softmax in the
//     exp2 domain with scale = sm_scale * log2(e) (:12), P cast to the input dtype, O += P KV,
//     glse = log2(l) + m * scale (:180-181);
//   combine (:186-221): lse = log2(sum_s 2^(glse_s - max)) + max, O = sum_s O_s * 2^(glse_s - lse).
//   Split partition (:140-144): the sequence's 64-token blocks are dealt out so the first
//   (blocks % num_split) splits take one extra block.
// The FP8 config stores the latent cache as OCP e4m3 with one fp32 scale: scores use
// (Q . K_fp8) * kv_scale and the output is (P . V_fp8) * kv_scale.
//
// gfx950 mapping of the split kernel:
//   * workgroup = (sequence, split, half of the query heads): 64 heads, 8 waves. The two halves of
//     a (sequence, split) are adjacent workgroup ids, so they run concurrently and the second read
//     of each KV tile is served by the Infinity Cache;
//   * wave (hg, dq): 32 heads (hg) and one quarter (dq) of the contraction dims: it computes the
//     partial S^T over d in [144*dq, 144*dq+144) and owns O^T rows d in [128*dq, 128*dq+128);
//     the four partial S^T tiles of a head group are summed through LDS;
//   * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16 (bf16/fp16): lanes index heads, so the
//     online softmax is lane-local; Q^T stays in VGPRs; P^T is the S^T accumulator rounded to the
//     input dtype; V^T is read from the row-major KV tile with ds_read_b64_tr_b16;
//   * 32-token KV tiles, gathered through the block table, fp8 decoded to bf16/fp16 (exact) while
//     staging into a double-buffered LDS tile; the next tile's global loads overlap the MFMAs.
#include "tlm_common.h"

#include <algorithm>
#include <mutex>

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int MLA_DV = 512, MLA_DPE = 64, MLA_D = MLA_DV + MLA_DPE;
constexpr int MLA_WAVES = 8;
constexpr int MLA_HEADS = 64;           // heads per workgroup
constexpr int MLA_BN = 32;              // tokens per KV tile
constexpr int MLA_PART_BLOCK = 64;      // default split partition granularity (reference block_N)
constexpr int KVP = MLA_D + 24;         // LDS pitch (halves): 1200 B rows
constexpr int QK_SUB = MLA_D / 16 / 4;  // 9 k-substeps of S^T per wave
constexpr int O_DT = MLA_DV / 4 / 32;   // 4 32-wide d tiles of O^T per wave

TLM_DEV s16x4 lds_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

template <bool BF16>
struct mla_mma;
template <>
struct mla_mma<false> {
  typedef f16x8 v8;
  static TLM_DEV f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct mla_mma<true> {
  typedef bf16x8 v8;
  static TLM_DEV f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

// 16 OCP e4m3 bytes -> 16 values of the MFMA input type (exact: every e4m3 value is
// representable in fp16 and bf16).
template <bool BF16>
TLM_DEV void fp8x16_to_h16(u32x4 in, u32x4& lo, u32x4& hi) {
  using H = h16<BF16>;
  u32x4 out[2];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)in[w], false);
    const f2 b = __builtin_amdgcn_cvt_pk_f32_fp8((int)in[w], true);
    out[w >> 1][(w & 1) * 2 + 0] = H::pack(a[0], a[1]);
    out[w >> 1][(w & 1) * 2 + 1] = H::pack(b[0], b[1]);
  }
  lo = out[0];
  hi = out[1];
}

// Token range [t0, t1) of split s of a sequence of L tokens: its blocks of `blk` tokens are dealt
// out so the first (blocks % num_split) splits take one extra (example_mla_decode_paged.py:
// 140-144). Empty when the sequence has fewer blocks than splits.
TLM_DEV void mla_split_range(int L, int num_split, int s, int blk, int& t0, int& t1) {
  const int total = (L + blk - 1) / blk;
  const int per = total / num_split, rem = total % num_split;
  const int nb = per + (s < rem ? 1 : 0);
  t0 = (per * s + min(s, rem)) * blk;
  t1 = min(t0 + nb * blk, L);
}

// KV_KIND: 0 = fp8 e4m3, 1 = same 16-bit type as Q.
template <bool BF16, int KV_KIND>
__global__ __launch_bounds__(64 * MLA_WAVES, 1) void mla_split_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ q_pe, int64_t q_stride,
    int64_t qpe_stride, const uint8_t* __restrict__ kv, const uint8_t* __restrict__ k_pe,
    int64_t kv_stride_b, int64_t kpe_stride_b, int64_t kv_rows,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ seqlens,
    float* __restrict__ ws_o, float* __restrict__ ws_lse,
    int Hq, int page, int max_pages, int num_split, float score_scale,
    const float* __restrict__ kv_scale, int part_block) {
  using MT = mla_mma<BF16>;
  using v8 = typename MT::v8;
  __shared__ __attribute__((aligned(16))) uint16_t sKV[2][MLA_BN * KVP];
  __shared__ float sRed[MLA_WAVES][16][64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hg = wave >> 2, dq = wave & 3;
  const int hhalves = Hq / MLA_HEADS;
  const int lin = blockIdx.x;
  const int hb = lin % hhalves;
  const int split = (lin / hhalves) % num_split;
  const int b = lin / (hhalves * num_split);
  // clamp to what the block table can address (a larger seqlen would index past the table)
  const int L = max(0, min(seqlens[b], max_pages * page));

  // token range of this split (reference partition over blocks of part_block tokens)
  int t_begin, t_end;
  mla_split_range(L, num_split, split, part_block, t_begin, t_end);
  const int nblk = t_end > t_begin ? (t_end - t_begin + MLA_BN - 1) / MLA_BN : 0;

  const float kvs = (KV_KIND == 0 && kv_scale) ? kv_scale[0] : 1.0f;
  const float c = score_scale * kvs;  // sm_scale * log2(e) * kv_scale

  const int ql = lane & 31, g = lane >> 5;
  const int head = hb * MLA_HEADS + hg * 32 + ql;
  // Q^T operand for this wave's 144 contraction dims
  v8 qreg[QK_SUB];
#pragma unroll
  for (int s = 0; s < QK_SUB; ++s) {
    const int d = 16 * (QK_SUB * dq + s) + 8 * g;
    const uint16_t* src = d < MLA_DV ? q + ((int64_t)b * Hq + head) * q_stride + d
                                     : q_pe + ((int64_t)b * Hq + head) * qpe_stride + (d - MLA_DV);
    qreg[s] = __builtin_bit_cast(v8, *(const u32x4*)src);
  }

  // staging: tile = 32 token rows; fp8 rows are 36 chunks of 16 bytes, 16-bit rows 72 chunks
  constexpr int CH = KV_KIND == 0 ? MLA_D / 16 : MLA_D / 8;
  constexpr int CH_DV = KV_KIND == 0 ? MLA_DV / 16 : MLA_DV / 8;
  constexpr int NPASS = (MLA_BN * CH + 64 * MLA_WAVES - 1) / (64 * MLA_WAVES);
  u32x4 rg[NPASS];
  auto load_tile = [&](int blk) {
    const int tok0 = t_begin + blk * MLA_BN;
#pragma unroll
    for (int p = 0; p < NPASS; ++p) {
      const int idx = tid + p * 64 * MLA_WAVES;
      rg[p] = u32x4{0, 0, 0, 0};
      if (idx < MLA_BN * CH) {
        const int r = idx / CH, ch = idx % CH;
        const int tok = tok0 + r;
        const int64_t row =
            tok < t_end
                ? (int64_t)block_table[(int64_t)b * max_pages + tok / page] * page + tok % page
                : -1;
        if (row >= 0 && row < kv_rows) {  // rows outside the pool read as zeros
          const uint8_t* src = ch < CH_DV ? kv + row * kv_stride_b + ch * 16
                                          : k_pe + row * kpe_stride_b + (ch - CH_DV) * 16;
          rg[p] = *(const u32x4*)src;
        }
      }
    }
  };
  auto store_tile = [&](int stage) {
#pragma unroll
    for (int p = 0; p < NPASS; ++p) {
      const int idx = tid + p * 64 * MLA_WAVES;
      if (idx < MLA_BN * CH) {
        const int r = idx / CH, ch = idx % CH;
        uint16_t* dst = &sKV[stage][r * KVP];
        if constexpr (KV_KIND == 0) {
          u32x4 lo, hi;
          fp8x16_to_h16<BF16>(rg[p], lo, hi);
          *(u32x4*)(dst + 16 * ch) = lo;
          *(u32x4*)(dst + 16 * ch + 8) = hi;
        } else {
          *(u32x4*)(dst + 8 * ch) = rg[p];
        }
      }
    }
  };

  f32x16 oacc[O_DT];
#pragma unroll
  for (int t = 0; t < O_DT; ++t) oacc[t] = f32x16{};
  float m_run = -INFINITY, l_part = 0.f;
  const int hh = lane >> 4, jj = lane & 15;

  if (nblk > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int blk = 0; blk < nblk; ++blk) {
    const int cur = blk & 1;
    const bool has_next = blk + 1 < nblk;
    if (has_next) load_tile(blk + 1);
    const uint16_t* kt = sKV[cur];
    // partial S^T[token][head] over this wave's 144 dims
    f32x16 sacc = f32x16{};
#pragma unroll
    for (int s = 0; s < QK_SUB; ++s) {
      const v8 a = *(const v8*)(kt + ql * KVP + 16 * (QK_SUB * dq + s) + 8 * g);
      sacc = MT::mma(a, qreg[s], sacc);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sRed[wave][i][lane] = sacc[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i)
      sacc[i] = sRed[4 * hg + 0][i][lane] + sRed[4 * hg + 1][i][lane] +
                sRed[4 * hg + 2][i][lane] + sRed[4 * hg + 3][i][lane];
    // softmax over this tile's tokens: token = tok0 + 8(i/4) + 4g + i%4
    const int tok0 = t_begin + blk * MLA_BN;
    float mloc = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float x = sacc[i] * c;
      if (tok0 + 8 * (i >> 2) + 4 * g + (i & 3) >= t_end) x = -INFINITY;
      sacc[i] = x;
      mloc = fmaxf(mloc, x);
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float m_new = fmaxf(m_run, mloc);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    m_run = m_new;
    float psum = 0.f;
    v8 pb[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      u32x4 pk;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p0 = fast_exp2(sacc[8 * s2 + 2 * e] - m_use);
        const float p1 = fast_exp2(sacc[8 * s2 + 2 * e + 1] - m_use);
        psum += p0 + p1;
        pk[e] = h16<BF16>::pack(p0, p1);
      }
      pb[s2] = __builtin_bit_cast(v8, pk);
    }
    l_part = l_part * alpha + psum;
#pragma unroll
    for (int dt = 0; dt < O_DT; ++dt) oacc[dt] *= alpha;
    // O^T[d][head] += V^T[d][token] P^T[token][head]
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int base = 16 * s2 + 4 * (hh >> 1) + (jj >> 2);
#pragma unroll
      for (int dt = 0; dt < O_DT; ++dt) {
        const uint16_t* p = kt + base * KVP + 128 * dq + 32 * dt + 16 * (hh & 1) + 4 * (jj & 3);
        const s16x4 lo = lds_tr16(p), hi = lds_tr16(p + 8 * KVP);
        const s16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        oacc[dt] = MT::mma(__builtin_bit_cast(v8, av), pb[s2], oacc[dt]);
      }
    }
    if (has_next) store_tile(cur ^ 1);
    __syncthreads();
  }

  // partial results: O_s (normalised by this split's l) and lse_s = m + log2(l), log2 domain
  const float l_tot = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  const int64_t slot = ((int64_t)b * Hq + head) * num_split + split;
  float* o = ws_o + slot * MLA_DV;
#pragma unroll
  for (int dt = 0; dt < O_DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = 128 * dq + 32 * dt + 8 * (i >> 2) + 4 * g + (i & 3);
      o[d] = oacc[dt][i] * inv;
    }
  if (dq == 0 && g == 0) ws_lse[slot] = l_tot > 0.f ? m_run + __log2f(l_tot) : -INFINITY;
}

// LSE combine: one workgroup of 128 threads per (sequence, head), 4 output values per thread.
template <bool OUT_BF16>
__global__ __launch_bounds__(128) void mla_combine_kernel(const float* __restrict__ ws_o,
                                                          const float* __restrict__ ws_lse,
                                                          uint16_t* __restrict__ out,
                                                          int num_split, const float* kv_scale,
                                                          int kv_is_fp8) {
  const int64_t bh = blockIdx.x;
  const float* lse = ws_lse + bh * num_split;
  float mx = -INFINITY;
  for (int s = 0; s < num_split; ++s) mx = fmaxf(mx, lse[s]);
  float sum = 0.f;
  for (int s = 0; s < num_split; ++s) sum += fast_exp2(lse[s] - mx);
  const float lse_tot = mx + __log2f(sum);
  const int d = threadIdx.x * 4;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < num_split; ++s) {
    if (lse[s] == -INFINITY) continue;
    const float w = fast_exp2(lse[s] - lse_tot);
    const f32x4 v = *(const f32x4*)(ws_o + (bh * num_split + s) * MLA_DV + d);
    acc += v * w;
  }
  const float kvs = (kv_is_fp8 && kv_scale) ? kv_scale[0] : 1.0f;
  acc *= kvs;
  using H = h16<OUT_BF16>;
  u32x2 pk = {H::pack(acc[0], acc[1]), H::pack(acc[2], acc[3])};
  *(u32x2*)(out + bh * MLA_DV + d) = pk;
}

// Combine of the split programs that keep their partials (example_mla_decode_paged.py:100-221,
// example_mla_decode.py): split s's normalised output (times kv_scale for fp8 KV) and log2
// sum-exp are stored rounded to the program's dtype in Output_partial [b, h, s, :] and glse
// [b, h, s], and Output is the combine of those stored values, as the program's combine kernel
// reads them back: O = sum_s O_s 2^(lse_s - lse), lse = log2 sum_s 2^(lse_s - max) + max. A split
// without tokens stores lse -inf and zeros (the reference divides 0 by 0 there). One workgroup
// per (sequence, head), 4 dims per thread.
// PK: storage of the partials, 0 fp16, 1 bf16, 2 fp32 (stored unrounded; part_store in
// tlm_common.h).

template <int PK, bool OUT_BF16>
__global__ __launch_bounds__(256) void mla_partial_combine(
    const float* __restrict__ ws_o, const float* __restrict__ ws_lse, void* __restrict__ glse,
    void* __restrict__ opart, uint16_t* __restrict__ out, int num_split, int dv,
    const float* kv_scale, int kv_is_fp8) {
  using PS = part_store<PK>;
  using HO = h16<OUT_BF16>;
  const int64_t bh = blockIdx.x;
  const int d = threadIdx.x * 4;
  const float* lse = ws_lse + bh * num_split;
  const float kvs = (kv_is_fp8 && kv_scale) ? kv_scale[0] : 1.0f;
  float M = -INFINITY, L = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < num_split; ++s) {
    const float l0 = lse[s];
    if (threadIdx.x == 0) PS::put_lse(glse, bh * num_split + s, l0);
    if (d >= dv) continue;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (l0 != -INFINITY) v = *(const f32x4*)(ws_o + (bh * num_split + s) * dv + d) * kvs;
    const f32x4 vr = PS::put4(opart, (bh * num_split + s) * dv + d, v);
    const float lr = PS::round(l0);  // the stored values, as read back
    if (lr != -INFINITY) {
      const float Mn = fmaxf(M, lr);
      const float a = fast_exp2(M - Mn), w = fast_exp2(lr - Mn);  // a = 0 while M = -inf
      L = L * a + w;
      acc = acc * a + vr * w;
      M = Mn;
    }
  }
  if (d >= dv) return;
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  *(u32x2*)(out + bh * dv + d) = u32x2{HO::pack(acc[0] * inv, acc[1] * inv),
                                       HO::pack(acc[2] * inv, acc[3] * inv)};
}

// ------------------------------------------------------------------------------------------------
// Paged gather: one 64-lane wave per token row; rows resolved through the block table exactly
// as the decode kernel resolves them (example_mla_decode_paged.py:62-63).
__global__ __launch_bounds__(256) void paged_gather_kernel(
    const uint8_t* __restrict__ kv, int64_t row_bytes, int64_t kv_rows,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ seqlens,
    const int64_t* __restrict__ cu, uint8_t* __restrict__ out, int64_t page, int64_t max_pages) {
  const int b = blockIdx.y;
  const int64_t L = max((int64_t)0, min((int64_t)seqlens[b], max_pages * page));
  const int lane = threadIdx.x & 63;
  for (int64_t j = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); j < L; j += (int64_t)gridDim.x * 4) {
    const int64_t row = (int64_t)block_table[b * max_pages + j / page] * page + j % page;
    const bool ok = row >= 0 && row < kv_rows;
    const uint8_t* src = kv + (ok ? row : 0) * row_bytes;
    uint8_t* dst = out + (cu[b] + j) * row_bytes;
    for (int64_t c = lane; c < row_bytes; c += 64) dst[c] = ok ? src[c] : (uint8_t)0;
  }
}

// ------------------------------------------------------------------------------------------------
// Generic decode for the shapes the matrix-core kernels do not take (head dims other than 512 +
// 64, head counts that are not a multiple of 64; e.g. the TPU demo's dim 32 + rope 4 over 8
// heads). Workgroup = one (sequence, head); 256 keys at a time: one thread per key for the
// score (dot product over dv + dpe), the online softmax in the exp2 domain with the workgroup's
// chunk maximum, P rounded to Q's dtype as the programs' P tiles are, then O accumulated with
// the threads spread over the dims. Correctness path for small shapes, not tuned.
constexpr int MLA_GEN_DV = 1024, MLA_GEN_DQK = MLA_GEN_DV + 256;

// Split mode (ws_o != nullptr, the split programs that keep their partials): workgroup =
// (sequence, head, split) over the split's token range; the normalised output (without
// kv_scale) goes to ws_o [b, h, s, :] and the log2 sum-exp to ws_lse [b, h, s].
template <bool BF16, int KV_KIND, bool O_BF16>
__global__ __launch_bounds__(256) void mla_generic_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ q_pe, int64_t qs, int64_t qpes,
    const uint8_t* __restrict__ kv, const uint8_t* __restrict__ k_pe, int64_t kvs_b,
    int64_t kpes_b, int64_t kv_rows, const int32_t* __restrict__ bt,
    const int32_t* __restrict__ sl, uint16_t* __restrict__ out, int Hq, int dv, int dpe,
    int page, int max_pages, float sc, const float* kv_scale, float* __restrict__ ws_o,
    float* __restrict__ ws_lse, int num_split, int part_block) {
  __shared__ float qf[MLA_GEN_DQK];
  __shared__ float pt[256];
  __shared__ int64_t rt[256];
  __shared__ float red[256];
  using HQ = h16<BF16>;
  const int tid = threadIdx.x;
  const bool split_mode = ws_o != nullptr;
  const int64_t bh = split_mode ? blockIdx.x / num_split : blockIdx.x;
  const int split = split_mode ? (int)(blockIdx.x % num_split) : 0;
  const int b = (int)(bh / Hq);
  const int dqk = dv + dpe;
  for (int d = tid; d < dqk; d += 256)
    qf[d] = HQ::to_f32(d < dv ? q[bh * qs + d] : q_pe[bh * qpes + (d - dv)]);
  const float kvs = (KV_KIND == 0 && kv_scale) ? kv_scale[0] : 1.0f;
  auto kv_val = [&](const uint8_t* row, int d) {
    if constexpr (KV_KIND == 0) {
      return __builtin_amdgcn_cvt_f32_fp8((int)row[d], 0);
    } else {
      return HQ::to_f32(((const uint16_t*)row)[d]);
    }
  };
  const int64_t lmax = (int64_t)max_pages * page;
  const int L_all = (int)max((int64_t)0, min((int64_t)sl[b], lmax));
  int c_lo = 0, L = L_all;  // token range [c_lo, L)
  if (split_mode) mla_split_range(L_all, num_split, split, part_block, c_lo, L);
  float m = -INFINITY, l = 0.f;
  float o[MLA_GEN_DV / 256] = {};
  auto block_reduce = [&](float v, bool is_max) {
    red[tid] = v;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
      if (tid < off) red[tid] = is_max ? fmaxf(red[tid], red[tid + off]) : red[tid] + red[tid + off];
      __syncthreads();
    }
    const float r = red[0];
    __syncthreads();
    return r;
  };
  __syncthreads();
  for (int c0 = c_lo; c0 < L; c0 += 256) {
    const int t = c0 + tid;
    float s = -INFINITY;
    int64_t row = -1;
    if (t < L) {
      row = (int64_t)bt[(int64_t)b * max_pages + t / page] * page + t % page;
      float acc = 0.f;
      if (row >= 0 && row < kv_rows) {  // rows outside the pool read as zeros
        const uint8_t* kr = kv + row * kvs_b;
        const uint8_t* pr = k_pe + row * kpes_b;
        for (int d = 0; d < dv; ++d) acc = fmaf(qf[d], kv_val(kr, d), acc);
        for (int d = 0; d < dpe; ++d) acc = fmaf(qf[dv + d], kv_val(pr, d), acc);
      } else {
        row = -1;
      }
      s = acc * kvs * sc;
    }
    const float m_new = fmaxf(m, block_reduce(s, true));
    const float alpha = __builtin_amdgcn_exp2f(m - m_new);
    const float p = t < L ? HQ::to_f32(HQ::from_f32(__builtin_amdgcn_exp2f(s - m_new))) : 0.f;
    pt[tid] = p;
    rt[tid] = row;
    l = l * alpha + block_reduce(p, false);
    m = m_new;
    const int n = min(256, L - c0);
#pragma unroll
    for (int k = 0; k < MLA_GEN_DV / 256; ++k) {
      const int d = tid + 256 * k;
      if (d >= dv) break;
      float acc = o[k] * alpha;
      for (int j = 0; j < n; ++j)
        if (rt[j] >= 0) acc = fmaf(pt[j], kv_val(kv + rt[j] * kvs_b, d), acc);
      o[k] = acc;
    }
    __syncthreads();
  }
  if (split_mode) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    const int64_t slot = bh * num_split + split;
#pragma unroll
    for (int k = 0; k < MLA_GEN_DV / 256; ++k) {
      const int d = tid + 256 * k;
      if (d < dv) ws_o[slot * dv + d] = o[k] * inv;
    }
    if (tid == 0) ws_lse[slot] = l > 0.f ? m + __log2f(l) : -INFINITY;
    return;
  }
  using HO = h16<O_BF16>;
  const float w = l > 0.f ? kvs / l : 0.f;
#pragma unroll
  for (int k = 0; k < MLA_GEN_DV / 256; ++k) {
    const int d = tid + 256 * k;
    if (d < dv) out[bh * dv + d] = (uint16_t)HO::from_f32(o[k] * w);
  }
}

template <bool BF16, int KV_KIND, bool O_BF16>
int launch_generic(const void* q, const void* q_pe, int64_t qs, int64_t qpes, const void* kv,
                   const void* k_pe, int64_t kvs_b, int64_t kpes_b, int64_t kv_rows,
                   const int32_t* bt, const int32_t* sl, void* o, int B, int Hq, int dv, int dpe,
                   int page, int max_pages, float sc, const float* kv_scale, hipStream_t st,
                   float* ws_o = nullptr, float* ws_lse = nullptr, int num_split = 1,
                   int part_block = MLA_PART_BLOCK) {
  const int64_t nwg = (int64_t)B * Hq * (ws_o ? num_split : 1);
  mla_generic_kernel<BF16, KV_KIND, O_BF16><<<(unsigned)nwg, 256, 0, st>>>(
      (const uint16_t*)q, (const uint16_t*)q_pe, qs, qpes, (const uint8_t*)kv,
      (const uint8_t*)k_pe, kvs_b, kpes_b, kv_rows, bt, sl, (uint16_t*)o, Hq, dv, dpe, page,
      max_pages, sc, kv_scale, ws_o, ws_lse, num_split, part_block);
  TLM_LAUNCH_CHECK("tlm_mla_decode (generic)");
  return TLM_OK;
}

template <bool BF16, int KV_KIND>
int launch_split(const void* q, const void* q_pe, int64_t qs, int64_t qpes, const void* kv,
                 const void* k_pe, int64_t kvs_b, int64_t kpes_b, int64_t kv_rows, const int32_t* bt,
                 const int32_t* sl, float* ws_o, float* ws_lse, int B, int Hq, int page,
                 int max_pages, int ns, float sc, const float* kv_scale, hipStream_t st,
                 int part_block = MLA_PART_BLOCK) {
  const int64_t nwg = (int64_t)B * ns * (Hq / MLA_HEADS);
  mla_split_kernel<BF16, KV_KIND><<<(unsigned)nwg, 64 * MLA_WAVES, 0, st>>>(
      (const uint16_t*)q, (const uint16_t*)q_pe, qs, qpes, (const uint8_t*)kv,
      (const uint8_t*)k_pe, kvs_b, kpes_b, kv_rows, bt, sl, ws_o, ws_lse, Hq, page, max_pages, ns, sc,
      kv_scale, part_block);
  TLM_LAUNCH_CHECK("tlm_mla_decode (split)");
  return TLM_OK;
}

}  // namespace

// FP8 path on the fp8 matrix cores (tlm_mla_fp8.hip); TLM_EUNSUPPORTED for shapes it does not take
size_t tlm_mla_fp8_workspace_bytes(int64_t B, int64_t Hq, int num_split);
bool tlm_mla_fp8_applies(int64_t B, int64_t Hq, int64_t page, int64_t max_pages,
                         int64_t kv_stride, int64_t kpe_stride);
int tlm_mla_fp8_launch(const void* q, const void* q_pe, int64_t q_stride, int64_t q_pe_stride,
                       const void* kv, const void* k_pe, int64_t kv_stride, int64_t kpe_stride,
                       int64_t kv_rows, const int32_t* block_table, const int32_t* seqlens,
                       void* o, void* ws, int64_t B, int64_t Hq, int64_t page, int64_t max_pages,
                       int num_split, float score_scale, const float* kv_scale, bool q_bf16,
                       bool o_bf16, void* stream);
size_t tlm_mla_fp8_segments_workspace_bytes(int64_t B, int64_t Hq, int num_split, int par);
int tlm_mla_fp8_launch_segments(const void* q, const void* q_pe, int64_t q_stride,
                                int64_t q_pe_stride, const void* kv, const void* k_pe,
                                int64_t kv_stride, int64_t kpe_stride, int64_t kv_rows,
                                const int32_t* block_table, const int32_t* seqlens, void* ws,
                                int64_t B, int64_t Hq, int64_t page, int64_t max_pages,
                                int num_split, int par, float score_scale,
                                const float* kv_scale, bool q_bf16, void* glse, void* o_partial,
                                int p_dtype, void* o, bool o_bf16, void* stream);

// Ranges of the split programs' fp8 path, whatever the program's split count: about 256
// workgroups over all head groups (f8_ranges(B, Hq, par) = B * par / head groups); the ranges
// are balanced over the B * num_split segments, so one range may hold several of them
static int mla_seg_par(int64_t B, int num_split) {
  (void)num_split;
  const int64_t fill = (256 + std::max<int64_t>(B, 1) - 1) / std::max<int64_t>(B, 1);
  return (int)std::min<int64_t>(64, fill);
}

// Workspace bytes of the two paths: the fp8 matrix-core path (fp8 KV, page a multiple of 64, Hq
// a multiple of 64; its own layout) and the split path (fp32 partial outputs + log2-sum-exp,
// one slot per (sequence, split, head)).
static size_t mla_split_workspace_bytes(int64_t B, int64_t Hq, int64_t dv, int num_split) {
  return (size_t)B * num_split * Hq * (dv + 1) * sizeof(float);
}

extern "C" size_t tlm_mla_workspace_bytes(int64_t B, int64_t Hq, int64_t dv, int num_split) {
  if (B <= 0 || Hq <= 0 || dv <= 0 || num_split <= 0) return 0;
  // the largest layout serves every path (the split programs' fp8 path included)
  return std::max({mla_split_workspace_bytes(B, Hq, dv, num_split),
                   tlm_mla_fp8_workspace_bytes(B, Hq, num_split),
                   tlm_mla_fp8_segments_workspace_bytes(B, Hq, num_split,
                                                        mla_seg_par(B, num_split))});
}

// The matrix-core kernels take dv = 512, dpe = 64, Hq a multiple of 64 and 16-byte aligned Q / KV
// rows; every other valid request runs the generic kernel.
static bool mla_fast_shape(const void* q, const void* q_pe, int64_t q_stride, int64_t q_pe_stride,
                           const void* kv, const void* k_pe, int64_t kv_stride,
                           int64_t kpe_stride, const void* o, int64_t Hq, int64_t dv, int64_t dpe,
                           int kv_dtype) {
  const int64_t kv_elt = kv_dtype == TLM_F8E4M3 ? 1 : 2;
  return dv == MLA_DV && dpe == MLA_DPE && Hq % MLA_HEADS == 0 && tlm_aligned(q, 16) &&
         tlm_aligned(q_pe, 16) && tlm_aligned(kv, 16) && tlm_aligned(k_pe, 16) &&
         q_stride % 8 == 0 && q_pe_stride % 8 == 0 && (kv_stride * kv_elt) % 16 == 0 &&
         (kpe_stride * kv_elt) % 16 == 0 && tlm_aligned(o, 8);
}

// Argument checks shared by tlm_mla_decode and tlm_mla_decode_noalloc (no HIP call).
static int mla_validate(const char* fn, const void* q, const void* q_pe, int64_t q_stride,
                        int64_t q_pe_stride, const void* kv, const void* k_pe, int64_t kv_stride,
                        int64_t kpe_stride, int64_t kv_rows, const int32_t* block_table,
                        const int32_t* seqlens, void* o, int64_t B, int64_t Hq, int64_t dv,
                        int64_t dpe, int64_t page, int64_t max_pages, int num_split,
                        int q_dtype, int kv_dtype, int o_dtype) {
  if (!q || !q_pe || !kv || !k_pe || !block_table || !seqlens || !o) {
    tlm_set_error("%s: null pointer argument", fn);
    return TLM_EINVAL;
  }
  if (B < 0 || B > (1 << 20) || Hq <= 0 || page <= 0 || max_pages <= 0 || num_split <= 0 ||
      num_split > 64 || page > (1 << 20) || max_pages > (1 << 20)) {
    tlm_set_error("%s: bad sizes B=%lld Hq=%lld page=%lld max_pages=%lld splits=%d", fn,
                  (long long)B, (long long)Hq, (long long)page, (long long)max_pages, num_split);
    return TLM_EINVAL;
  }
  if (max_pages * page > INT32_MAX) {
    tlm_set_error("%s: max_pages * page exceeds the int32 token range", fn);
    return TLM_EINVAL;
  }
  if (dv < 1 || dv > MLA_GEN_DV || dpe < 0 || dpe > MLA_GEN_DQK - MLA_GEN_DV || Hq > 4096) {
    tlm_set_error("%s: head dims dv in [1, %d], dpe in [0, %d] and at most 4096 heads "
                  "(got dv=%lld dpe=%lld Hq=%lld)", fn, MLA_GEN_DV, MLA_GEN_DQK - MLA_GEN_DV,
                  (long long)dv, (long long)dpe, (long long)Hq);
    return TLM_EUNSUPPORTED;
  }
  if (q_stride < dv || q_pe_stride < dpe || kv_stride < dv || kpe_stride < dpe || kv_rows < 0) {
    tlm_set_error("%s: row strides smaller than the row widths", fn);
    return TLM_EINVAL;
  }
  if ((q_dtype != TLM_BF16 && q_dtype != TLM_F16) || (o_dtype != TLM_BF16 && o_dtype != TLM_F16) ||
      (kv_dtype != TLM_F8E4M3 && kv_dtype != q_dtype)) {
    tlm_set_error("%s: dtype combination q=%d kv=%d o=%d unsupported (kv must be "
                  "fp8 e4m3 or Q's dtype)", fn, q_dtype, kv_dtype, o_dtype);
    return TLM_EUNSUPPORTED;
  }
  const size_t kv_elt = kv_dtype == TLM_F8E4M3 ? 1 : 2;
  if (!tlm_aligned(q, 2) || !tlm_aligned(q_pe, 2) || !tlm_aligned(kv, kv_elt) ||
      !tlm_aligned(k_pe, kv_elt) || !tlm_aligned(o, 2)) {
    tlm_set_error("%s: misaligned Q/KV/O pointer", fn);
    return TLM_EINVAL;
  }
  if (B > 0 && kv_rows < 1) {
    tlm_set_error("%s: empty KV pool", fn);
    return TLM_EINVAL;
  }
  return TLM_OK;
}

// The decode proper on validated arguments. ws_bytes is checked against the need of the path
// taken (ws is 16-byte aligned).
static int mla_run(const char* fn, const void* q, const void* q_pe, int64_t q_stride,
                   int64_t q_pe_stride, const void* kv, const void* k_pe, int64_t kv_stride,
                   int64_t kpe_stride, int64_t kv_rows, const int32_t* block_table,
                   const int32_t* seqlens, void* o, void* ws, size_t ws_bytes, int64_t B,
                   int64_t Hq, int64_t dv, int64_t dpe, int64_t page, int64_t max_pages,
                   int num_split, float sm_scale, const float* kv_scale, int q_dtype,
                   int kv_dtype, int o_dtype, void* stream, void* glse = nullptr,
                   void* opart = nullptr, int part_block = MLA_PART_BLOCK,
                   int p_dtype = TLM_F16) {
  if (B == 0) return TLM_OK;
  const float sc = (float)((double)sm_scale * 1.4426950408889634);
  const bool partials = glse != nullptr && opart != nullptr;
  const bool fast = mla_fast_shape(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride,
                                   kpe_stride, o, Hq, dv, dpe, kv_dtype);
  if (partials && fast && kv_dtype == TLM_F8E4M3 && part_block == 64 &&
      dv == MLA_DV && tlm_mla_fp8_applies(B, Hq, page, max_pages, kv_stride, kpe_stride) &&
      tlm_mla_fp8_segments_workspace_bytes(B, Hq, num_split, mla_seg_par(B, num_split)) > 0 &&
      ws_bytes >= tlm_mla_fp8_segments_workspace_bytes(B, Hq, num_split,
                                                       mla_seg_par(B, num_split))) {
    // the program's partition (64-token blocks) on the balanced 128-head fp8 decode: each split
    // is a segment of its sequence, then the partials and Output as above
    const int rc = tlm_mla_fp8_launch_segments(
        q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride, kpe_stride, kv_rows, block_table,
        seqlens, ws, B, Hq, page, max_pages, num_split, mla_seg_par(B, num_split), sc, kv_scale,
        q_dtype == TLM_BF16, glse, opart, p_dtype, o, o_dtype == TLM_BF16, stream);
    if (rc != TLM_EUNSUPPORTED) return rc;
  }
  if (partials) {
    // the program's own split partition, its partials stored, Output from the stored values
    if (ws_bytes < mla_split_workspace_bytes(B, Hq, dv, num_split)) {
      tlm_set_error("%s: %zu bytes of workspace, %zu required", fn, ws_bytes,
                    mla_split_workspace_bytes(B, Hq, dv, num_split));
      return TLM_EWORKSPACE;
    }
    hipStream_t st = (hipStream_t)stream;
    float* ws_o = (float*)ws;
    float* ws_lse = ws_o + (size_t)B * Hq * num_split * dv;
    const bool bq = q_dtype == TLM_BF16;
    const bool f8 = kv_dtype == TLM_F8E4M3;
    const int b = (int)B, h = (int)Hq, pg = (int)page, mp = (int)max_pages;
    const int64_t kb = f8 ? 1 : 2;
    int rc;
    if (fast) {
      rc = bq ? (f8 ? launch_split<true, 0>(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride,
                                            kpe_stride, kv_rows, block_table, seqlens, ws_o,
                                            ws_lse, b, h, pg, mp, num_split, sc, kv_scale, st,
                                            part_block)
                    : launch_split<true, 1>(q, q_pe, q_stride, q_pe_stride, kv, k_pe,
                                            kv_stride * 2, kpe_stride * 2, kv_rows, block_table,
                                            seqlens, ws_o, ws_lse, b, h, pg, mp, num_split, sc,
                                            kv_scale, st, part_block))
              : (f8 ? launch_split<false, 0>(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride,
                                             kpe_stride, kv_rows, block_table, seqlens, ws_o,
                                             ws_lse, b, h, pg, mp, num_split, sc, kv_scale, st,
                                             part_block)
                    : launch_split<false, 1>(q, q_pe, q_stride, q_pe_stride, kv, k_pe,
                                             kv_stride * 2, kpe_stride * 2, kv_rows, block_table,
                                             seqlens, ws_o, ws_lse, b, h, pg, mp, num_split, sc,
                                             kv_scale, st, part_block));
    } else {
#define TLM_MLA_GENS(BQ, KK)                                                                       \
  launch_generic<BQ, KK, false>(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride * kb,         \
                                kpe_stride * kb, kv_rows, block_table, seqlens, o, b, h, (int)dv, \
                                (int)dpe, pg, mp, sc, kv_scale, st, ws_o, ws_lse, num_split,      \
                                part_block)
      rc = bq ? (f8 ? TLM_MLA_GENS(true, 0) : TLM_MLA_GENS(true, 1))
              : (f8 ? TLM_MLA_GENS(false, 0) : TLM_MLA_GENS(false, 1));
#undef TLM_MLA_GENS
    }
    if (rc) return rc;
    const unsigned nthr = (unsigned)(((dv / 4) + 63) / 64 * 64);
    const unsigned nwg = (unsigned)(B * Hq);
    auto comb = [&](auto kern) {
      kern<<<nwg, nthr, 0, st>>>(ws_o, ws_lse, glse, opart, (uint16_t*)o, num_split, (int)dv,
                                 kv_scale, f8 ? 1 : 0);
    };
    const bool ob = o_dtype == TLM_BF16;
    if (p_dtype == TLM_F32)
      ob ? comb(mla_partial_combine<2, true>) : comb(mla_partial_combine<2, false>);
    else if (p_dtype == TLM_BF16)
      ob ? comb(mla_partial_combine<1, true>) : comb(mla_partial_combine<1, false>);
    else
      ob ? comb(mla_partial_combine<0, true>) : comb(mla_partial_combine<0, false>);
    TLM_LAUNCH_CHECK("tlm_mla_decode (partial combine)");
    return TLM_OK;
  }
  if (!fast) {
    hipStream_t st = (hipStream_t)stream;
    const int64_t kb = kv_dtype == TLM_F8E4M3 ? 1 : 2;
    const int b = (int)B, h = (int)Hq, pg = (int)page, mp = (int)max_pages;
    const int v = (int)dv, pe = (int)dpe;
    const bool bq = q_dtype == TLM_BF16, bo = o_dtype == TLM_BF16;
#define TLM_MLA_GEN(BQ, KK, BO)                                                                    \
  launch_generic<BQ, KK, BO>(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride * kb,            \
                             kpe_stride * kb, kv_rows, block_table, seqlens, o, b, h, v, pe, pg,  \
                             mp, sc, kv_scale, st)
    if (kv_dtype == TLM_F8E4M3)
      return bq ? (bo ? TLM_MLA_GEN(true, 0, true) : TLM_MLA_GEN(true, 0, false))
                : (bo ? TLM_MLA_GEN(false, 0, true) : TLM_MLA_GEN(false, 0, false));
    return bq ? (bo ? TLM_MLA_GEN(true, 1, true) : TLM_MLA_GEN(true, 1, false))
              : (bo ? TLM_MLA_GEN(false, 1, true) : TLM_MLA_GEN(false, 1, false));
#undef TLM_MLA_GEN
  }
  if (kv_dtype == TLM_F8E4M3) {
    const size_t need = tlm_mla_fp8_workspace_bytes(B, Hq, num_split);
    if (need > 0 && need <= ws_bytes) {
      const int rc = tlm_mla_fp8_launch(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride,
                                        kpe_stride, kv_rows, block_table, seqlens, o, ws, B, Hq,
                                        page, max_pages, num_split, sc, kv_scale,
                                        q_dtype == TLM_BF16, o_dtype == TLM_BF16, stream);
      if (rc != TLM_EUNSUPPORTED) return rc;
    }
  }
  if (ws_bytes < mla_split_workspace_bytes(B, Hq, dv, num_split)) {
    tlm_set_error("%s: %zu bytes of workspace, %zu required", fn, ws_bytes,
                  std::max(mla_split_workspace_bytes(B, Hq, dv, num_split),
                           kv_dtype == TLM_F8E4M3 ? tlm_mla_fp8_workspace_bytes(B, Hq, num_split)
                                                  : (size_t)0));
    return TLM_EWORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  float* ws_o = (float*)ws;
  float* ws_lse = ws_o + (size_t)B * Hq * num_split * dv;
  const bool bf = q_dtype == TLM_BF16;
  const int b = (int)B, h = (int)Hq, pg = (int)page, mp = (int)max_pages;
  int rc;
  if (kv_dtype == TLM_F8E4M3)
    rc = bf ? launch_split<true, 0>(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride,
                                    kpe_stride, kv_rows, block_table, seqlens, ws_o, ws_lse, b, h, pg, mp,
                                    num_split, sc, kv_scale, st)
            : launch_split<false, 0>(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride,
                                     kpe_stride, kv_rows, block_table, seqlens, ws_o, ws_lse, b, h, pg, mp,
                                     num_split, sc, kv_scale, st);
  else
    rc = bf ? launch_split<true, 1>(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride * 2,
                                    kpe_stride * 2, kv_rows, block_table, seqlens, ws_o, ws_lse, b, h, pg,
                                    mp, num_split, sc, kv_scale, st)
            : launch_split<false, 1>(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride * 2,
                                     kpe_stride * 2, kv_rows, block_table, seqlens, ws_o, ws_lse, b, h, pg,
                                     mp, num_split, sc, kv_scale, st);
  if (rc) return rc;
  const unsigned ncomb = (unsigned)(B * Hq);
  if (o_dtype == TLM_BF16)
    mla_combine_kernel<true><<<ncomb, 128, 0, st>>>(ws_o, ws_lse, (uint16_t*)o, num_split,
                                                    kv_scale, kv_dtype == TLM_F8E4M3);
  else
    mla_combine_kernel<false><<<ncomb, 128, 0, st>>>(ws_o, ws_lse, (uint16_t*)o, num_split,
                                                     kv_scale, kv_dtype == TLM_F8E4M3);
  TLM_LAUNCH_CHECK("tlm_mla_decode (combine)");
  return TLM_OK;
}

extern "C" int tlm_mla_decode(const void* q, const void* q_pe, int64_t q_stride,
                              int64_t q_pe_stride, const void* kv, const void* k_pe,
                              int64_t kv_stride, int64_t kpe_stride, int64_t kv_rows,
                              const int32_t* block_table, const int32_t* seqlens, void* o,
                              void* ws, size_t ws_bytes,
                              int64_t B, int64_t Hq, int64_t dv, int64_t dpe, int64_t page,
                              int64_t max_pages, int num_split, float sm_scale,
                              const float* kv_scale, int q_dtype, int kv_dtype, int o_dtype,
                              void* stream) {
  const char* fn = "tlm_mla_decode";
  int rc = mla_validate(fn, q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride, kpe_stride,
                        kv_rows, block_table, seqlens, o, B, Hq, dv, dpe, page, max_pages,
                        num_split, q_dtype, kv_dtype, o_dtype);
  if (rc) return rc;
  if (ws_bytes < tlm_mla_workspace_bytes(B, Hq, dv, num_split) || (B > 0 && !ws)) {
    tlm_set_error("tlm_mla_decode: workspace of %zu bytes is smaller than the %zu required",
                  ws_bytes, tlm_mla_workspace_bytes(B, Hq, dv, num_split));
    return TLM_EWORKSPACE;
  }
  if (!tlm_aligned(ws, 16)) {
    tlm_set_error("tlm_mla_decode: workspace must be 16-byte aligned");
    return TLM_EUNSUPPORTED;
  }
  return mla_run(fn, q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride, kpe_stride, kv_rows,
                 block_table, seqlens, o, ws, ws_bytes, B, Hq, dv, dpe, page, max_pages, num_split,
                 sm_scale, kv_scale, q_dtype, kv_dtype, o_dtype, stream);
}

extern "C" int tlm_mla_decode_ex(const void* q, const void* q_pe, int64_t q_stride,
                                 int64_t q_pe_stride, const void* kv, const void* k_pe,
                                 int64_t kv_stride, int64_t kpe_stride, int64_t kv_rows,
                                 const int32_t* block_table, const int32_t* seqlens, void* o,
                                 void* ws, size_t ws_bytes, int64_t B, int64_t Hq, int64_t dv,
                                 int64_t dpe, int64_t page, int64_t max_pages, int num_split,
                                 float sm_scale, const float* kv_scale, int q_dtype, int kv_dtype,
                                 int o_dtype, void* glse, void* o_partial, int64_t part_block,
                                 int p_dtype, void* stream) {
  const char* fn = "tlm_mla_decode_ex";
  if (!glse && !o_partial)
    return tlm_mla_decode(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride, kpe_stride,
                          kv_rows, block_table, seqlens, o, ws, ws_bytes, B, Hq, dv, dpe, page,
                          max_pages, num_split, sm_scale, kv_scale, q_dtype, kv_dtype, o_dtype,
                          stream);
  int rc = mla_validate(fn, q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride, kpe_stride,
                        kv_rows, block_table, seqlens, o, B, Hq, dv, dpe, page, max_pages,
                        num_split, q_dtype, kv_dtype, o_dtype);
  if (rc) return rc;
  if (part_block < 1 || part_block > (1 << 20) ||
      (p_dtype != TLM_F16 && p_dtype != TLM_BF16 && p_dtype != TLM_F32)) {
    tlm_set_error("%s: part_block %lld must be in [1, 2^20] and p_dtype F16, BF16 or F32", fn,
                  (long long)part_block);
    return TLM_EINVAL;
  }
  const size_t pe = p_dtype == TLM_F32 ? 4 : 2;
  if (!glse || !o_partial || !tlm_aligned(glse, pe) || !tlm_aligned(o_partial, 4 * pe)) {
    tlm_set_error("%s: glse and o_partial must both be given (aligned to 1 and 4 elements)", fn);
    return TLM_EINVAL;
  }
  if (dv % 4) {
    tlm_set_error("%s: partials need dv a multiple of 4 (got %lld)", fn, (long long)dv);
    return TLM_EUNSUPPORTED;
  }
  if ((int64_t)B * Hq * num_split > INT32_MAX) {
    tlm_set_error("%s: problem too large", fn);
    return TLM_EINVAL;
  }
  if (B > 0 && (!ws || !tlm_aligned(ws, 16))) {
    tlm_set_error("%s: workspace must be non-null and 16-byte aligned", fn);
    return TLM_EINVAL;
  }
  return mla_run(fn, q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride, kpe_stride, kv_rows,
                 block_table, seqlens, o, ws, ws_bytes, B, Hq, dv, dpe, page, max_pages, num_split,
                 sm_scale, kv_scale, q_dtype, kv_dtype, o_dtype, stream, glse, o_partial,
                 (int)part_block, p_dtype);
}

// ---- allocation-free variant ------------------------------------------------------------------
// The scratch of tlm_mla_decode_noalloc: a file-scope device array, one instance per GPU (each
// device that loads this code object holds its own copy at its own address until the process
// ends). In host code `scratch` only names the symbol: its device address is looked up once per
// device with hipGetSymbolAddress and kept in g_scratch_ptr, which is what kernels receive.
static __device__ __align__(256) uint8_t scratch[TLM_MLA_SCRATCH_BYTES];

namespace {
constexpr int kScratchDevices = 64;
std::once_flag g_scratch_once[kScratchDevices];
void* g_scratch_ptr[kScratchDevices];
hipError_t g_scratch_err[kScratchDevices];
}  // namespace

// Resolve this device's scratch address (device `dev` must be current). Called from tlm_init and,
// for callers that skip tlm_init, from the entry point's first call on a device.
int tlm_mla_scratch_setup(int dev) {
  if (dev < 0 || dev >= kScratchDevices) {
    tlm_set_error("tlm_mla_decode_noalloc: device index %d out of range", dev);
    return TLM_EINVAL;
  }
  std::call_once(g_scratch_once[dev], [dev]() {
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? p : nullptr;
  });
  if (g_scratch_err[dev] != hipSuccess)
    return tlm_hip_fail(g_scratch_err[dev], "hipGetSymbolAddress(scratch)");
  return TLM_OK;
}

extern "C" size_t tlm_mla_scratch_bytes(void) { return TLM_MLA_SCRATCH_BYTES; }

extern "C" int tlm_mla_decode_noalloc(const void* q, const void* q_pe, int64_t q_stride,
                                      int64_t q_pe_stride, const void* kv, const void* k_pe,
                                      int64_t kv_stride, int64_t kpe_stride, int64_t kv_rows,
                                      const int32_t* block_table, const int32_t* seqlens, void* o,
                                      int64_t B, int64_t Hq, int64_t dv, int64_t dpe,
                                      int64_t page, int64_t max_pages, int num_split,
                                      float sm_scale, const float* kv_scale, int q_dtype,
                                      int kv_dtype, int o_dtype, void* stream) {
  const char* fn = "tlm_mla_decode_noalloc";
  int rc = mla_validate(fn, q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride, kpe_stride,
                        kv_rows, block_table, seqlens, o, B, Hq, dv, dpe, page, max_pages,
                        num_split, q_dtype, kv_dtype, o_dtype);
  if (rc) return rc;
  // the path taken must fit the scratch (checked before any HIP call)
  const bool fast = mla_fast_shape(q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride,
                                   kpe_stride, o, Hq, dv, dpe, kv_dtype);
  const bool fp8 = fast && kv_dtype == TLM_F8E4M3 &&
                   tlm_mla_fp8_applies(B, Hq, page, max_pages, kv_stride, kpe_stride);
  const size_t need = !fast ? 0
                      : fp8 ? tlm_mla_fp8_workspace_bytes(B, Hq, num_split)
                            : mla_split_workspace_bytes(B, Hq, dv, num_split);
  if (need > TLM_MLA_SCRATCH_BYTES) {
    tlm_set_error("%s: this call needs %zu bytes of scratch, more than the library's %zu "
                  "(lower num_split or the batch, or use tlm_mla_decode with a workspace)", fn,
                  need, (size_t)TLM_MLA_SCRATCH_BYTES);
    return TLM_EWORKSPACE;
  }
  if (B == 0) return TLM_OK;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return tlm_hip_fail(e, "hipGetDevice");
  rc = tlm_mla_scratch_setup(dev);
  if (rc) return rc;
  return mla_run(fn, q, q_pe, q_stride, q_pe_stride, kv, k_pe, kv_stride, kpe_stride, kv_rows,
                 block_table, seqlens, o, g_scratch_ptr[dev], TLM_MLA_SCRATCH_BYTES, B, Hq, dv,
                 dpe, page, max_pages, num_split, sm_scale, kv_scale, q_dtype, kv_dtype, o_dtype,
                 stream);
}

extern "C" int tlm_paged_gather(const void* kv_bytes, int64_t row_bytes, int64_t kv_rows,
                                const int32_t* block_table, const int32_t* seqlens,
                                const int64_t* cu_seqlens, void* out, int64_t B, int64_t page,
                                int64_t max_pages, void* stream) {
  if (!kv_bytes || !block_table || !seqlens || !cu_seqlens || !out) {
    tlm_set_error("tlm_paged_gather: null pointer argument");
    return TLM_EINVAL;
  }
  if (B < 0 || B > 65535 || row_bytes <= 0 || page <= 0 || max_pages <= 0 || kv_rows < 0) {
    tlm_set_error("tlm_paged_gather: bad sizes");
    return TLM_EINVAL;
  }
  if (B == 0) return TLM_OK;
  dim3 grid(256, (unsigned)B);
  paged_gather_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)kv_bytes, row_bytes, kv_rows, block_table, seqlens, cu_seqlens, (uint8_t*)out, page,
      max_pages);
  TLM_LAUNCH_CHECK("tlm_paged_gather");
  return TLM_OK;
}
