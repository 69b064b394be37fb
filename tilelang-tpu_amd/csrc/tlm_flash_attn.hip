// FlashAttention forward (BSHD) on gfx950 MFMA.
//
// Reference program: tpu_demo/flashattn/tpu_test_flashattn_bf16.py:14-135 — per Q tile, loop over
// KV tiles: S = Q K^T (ppl_gemm transpose_B), online softmax (m = rowmax, alpha = exp((m_prev-m)*sc),
// P = exp((S-m)*sc), l = l*alpha + rowsum(P)), P cast to the input dtype, O = O*alpha + P V,
// finally O / l. Causal keeps key j <= query i (element mask of ref_program :171-182 and of the
// upstream example_mha_fwd_bshd.py:50-53).
//
// Layout of the work on gfx950:
//   * workgroup = 8 waves = 256 queries of one (batch, head); wave w owns 32 queries;
//   * scores are computed transposed, S^T = K * Q^T, with v_mfma_f32_32x32x16: the accumulator
//     layout then gives every lane ONE query (lane % 32) and 16 keys, so the row max / row sum of
//     the online softmax are lane-local plus one xor-32 shuffle;
//   * the output is accumulated transposed too, O^T = V^T * P^T: P^T is the S^T accumulator
//     itself (rounded to bf16/fp16 in registers, no LDS round trip) and alpha rescales stay
//     lane-local. V^T comes from the row-major V tile in LDS through ds_read_b64_tr_b16;
//   * Q stays in VGPRs for the whole loop (B operand of S^T); K and V tiles of 64 keys are
//     double-buffered in LDS, the next tile's global loads in flight during the current MFMAs;
//   * softmax runs in the exp2 domain with sm_scale*log2(e) folded into one multiply;
//   * causal: a wave skips key tiles above its diagonal, masks only the tile it crosses, and
//     workgroups are issued heaviest query tile first.
#include "tlm_common.h"

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int FA_WAVES = 8;
constexpr int BQ = 32 * FA_WAVES;  // queries per workgroup
constexpr int BKV = 64;            // keys per tile

TLM_DEV s16x4 lds_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
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

template <bool BF16, bool CAUSAL, int D>
__global__ __launch_bounds__(64 * FA_WAVES, 1) void fa_fwd(const uint16_t* __restrict__ Q,
                                                          const uint16_t* __restrict__ K,
                                                          const uint16_t* __restrict__ V,
                                                          uint16_t* __restrict__ O, int B, int S,
                                                          int H, float scale_log2) {
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
  const int64_t row_stride = (int64_t)H * D;  // elements between consecutive tokens
  const uint16_t* Qb = Q + ((int64_t)b * S * H + h) * D;
  const uint16_t* Kb = K + ((int64_t)b * S * H + h) * D;
  const uint16_t* Vb = V + ((int64_t)b * S * H + h) * D;

  const int ql = lane & 31, g = lane >> 5;
  const int qw0 = q0 + 32 * wave;  // first query of this wave
  const int my_q = qw0 + ql;

  // Q^T operand: lane holds query my_q, d = 16*ds + 8*g .. +7
  v8 qreg[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    u32x4 v = {0, 0, 0, 0};
    if (my_q < S) v = *(const u32x4*)(Qb + (int64_t)my_q * row_stride + 16 * ds + 8 * g);
    qreg[ds] = __builtin_bit_cast(v8, v);
  }

  const int kv_end = CAUSAL ? min(S, q0 + BQ) : S;
  const int nblk = (kv_end + BKV - 1) / BKV;
  const int wave_qmax = min(qw0 + 31, S - 1);  // < qw0 when the whole wave is past S

  u32x4 rk[LD_ITERS], rv[LD_ITERS];
  auto load_tile = [&](int j) {
#pragma unroll
    for (int p = 0; p < LD_ITERS; ++p) {
      const int idx = tid + p * 64 * FA_WAVES;
      const int r = idx / CH, c = (idx % CH) * 8;
      const int key = j * BKV + r;
      if (key < S) {
        rk[p] = *(const u32x4*)(Kb + (int64_t)key * row_stride + c);
        rv[p] = *(const u32x4*)(Vb + (int64_t)key * row_stride + c);
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
    const bool active = (qw0 < S) && (!CAUSAL || k0 <= wave_qmax);
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
      // scale, mask, row max (keys of this lane: 32t + 8(i/4) + 4g + i%4)
      const bool need_mask = (CAUSAL && k0 + BKV - 1 > qw0) || (k0 + BKV > S);
      float mloc = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float x = sacc[t][i] * scale_log2;
          if (need_mask) {
            const int key = k0 + 32 * t + 8 * (i >> 2) + 4 * g + (i & 3);
            if (key >= S || (CAUSAL && key > my_q)) x = -INFINITY;
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
      v8 pb[2][2];
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
  uint16_t* Ob = O + ((int64_t)b * S * H + h) * D;
#pragma unroll
  for (int it = 0; it < 32 * CH / 64; ++it) {
    const int idx = lane + 64 * it;
    const int r = idx / CH, c = (idx % CH) * 8;
    const int q = qw0 + r;
    if (q < S) *(u32x4*)(Ob + (int64_t)q * row_stride + c) = *(const u32x4*)(stage + r * OP + c);
  }
}

template <bool BF16, bool CAUSAL, int D>
int launch(const void* q, const void* k, const void* v, void* o, int B, int S, int H, float sc,
           hipStream_t st) {
  const int64_t nwg = (int64_t)((S + BQ - 1) / BQ) * B * H;
  if (nwg > INT32_MAX) {
    tlm_set_error("tlm_flash_attn_fwd: problem too large");
    return TLM_EINVAL;
  }
  fa_fwd<BF16, CAUSAL, D><<<(unsigned)nwg, 64 * FA_WAVES, 0, st>>>(
      (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, B, S, H, sc);
  TLM_LAUNCH_CHECK("tlm_flash_attn_fwd");
  return TLM_OK;
}

template <bool BF16>
int by_shape(const void* q, const void* k, const void* v, void* o, int B, int S, int H, int D,
             bool causal, float sc, hipStream_t st) {
  if (D == 128)
    return causal ? launch<BF16, true, 128>(q, k, v, o, B, S, H, sc, st)
                  : launch<BF16, false, 128>(q, k, v, o, B, S, H, sc, st);
  return causal ? launch<BF16, true, 64>(q, k, v, o, B, S, H, sc, st)
                : launch<BF16, false, 64>(q, k, v, o, B, S, H, sc, st);
}

}  // namespace

extern "C" int tlm_flash_attn_fwd(const void* q, const void* k, const void* v, void* o,
                                  int64_t B, int64_t S, int64_t H, int64_t D, int causal,
                                  float sm_scale, int dtype, void* stream) {
  if (!q || !k || !v || !o) {
    tlm_set_error("tlm_flash_attn_fwd: null pointer argument");
    return TLM_EINVAL;
  }
  if (B < 0 || S < 0 || H < 0 || B > 65535 || H > 65535 || S > (1 << 24)) {
    tlm_set_error("tlm_flash_attn_fwd: bad shape");
    return TLM_EINVAL;
  }
  if (D != 128 && D != 64) {
    tlm_set_error("tlm_flash_attn_fwd: head dim %lld unsupported (64 or 128)", (long long)D);
    return TLM_EUNSUPPORTED;
  }
  if (dtype != TLM_BF16 && dtype != TLM_F16) {
    tlm_set_error("tlm_flash_attn_fwd: dtype %d unsupported (BF16 or F16)", dtype);
    return TLM_EUNSUPPORTED;
  }
  if (!(sm_scale > 0.f) || !__builtin_isfinite(sm_scale)) {
    tlm_set_error("tlm_flash_attn_fwd: sm_scale must be positive and finite");
    return TLM_EINVAL;
  }
  if (!tlm_aligned(q, 16) || !tlm_aligned(k, 16) || !tlm_aligned(v, 16) || !tlm_aligned(o, 16)) {
    tlm_set_error("tlm_flash_attn_fwd: tensors must be 16-byte aligned");
    return TLM_EINVAL;
  }
  if (B == 0 || S == 0 || H == 0) return TLM_OK;
  const float sc = (float)((double)sm_scale * 1.4426950408889634);
  hipStream_t st = (hipStream_t)stream;
  return dtype == TLM_BF16 ? by_shape<true>(q, k, v, o, (int)B, (int)S, (int)H, (int)D,
                                            causal != 0, sc, st)
                           : by_shape<false>(q, k, v, o, (int)B, (int)S, (int)H, (int)D,
                                             causal != 0, sc, st);
}
