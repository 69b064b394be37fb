// Elementwise tile programs: the stand-alone T.ppl_* elementwise programs of the TPU demos
// (tpu_demo/ppl/test/exp.py, mul_N_1.py, elementwise_c.py; tpu_demo/ppl/elementwise_add_kernel/
// elementwise_add.py) and any other chain of ppl_add / ppl_sub / ppl_mul / ppl_div (second operand
// broadcast from an (M, 1) tile, codegen_ppl.cc:874-883), ppl_add_C / ppl_mul_C, ppl_exp2 (natural
// exponential), ppl_rsqrt and ppl_sigmoid between tile copies.
//
// The recogniser evaluates the program's tile ops symbolically into a short register program
// (include/tlmi355x.h: tlm_elementwise); this kernel runs it for every element of the [rows,
// cols] output domain. The instruction stream is a kernel argument, so its fetch and the op
// dispatch are scalar (wave-uniform) work; the per-element work is the VALU arithmetic and the
// HBM loads / stores, which are coalesced along the rows.
#include "tlm_common.h"

#include <algorithm>

namespace {

struct EwArgs {
  const void* in[TLM_EW_MAX_IN];
  void* out[TLM_EW_MAX_OUT];
  int in_dt[TLM_EW_MAX_IN];
  int in_bc[TLM_EW_MAX_IN];
  int out_dt[TLM_EW_MAX_OUT];
  uint32_t code[TLM_EW_MAX_CODE];
  float cst[TLM_EW_MAX_CONST];
  int n_code;
  int64_t rows, cols;
};

TLM_DEV float ew_to_f32(const void* p, int64_t idx, int dt) {
  if (dt == TLM_F32) return ((const float*)p)[idx];
  const uint32_t b = ((const uint16_t*)p)[idx];
  return dt == TLM_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}
TLM_DEV float ew_round(float v, int dt) {  // round to a 16-bit tile dtype (RNE) and back
  if (dt == TLM_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  if (dt == TLM_F16) return f16_bits_to_f32(f32_to_f16_bits(v));
  return v;
}

// Register slots addressed with wave-uniform indices: switch statements keep them in VGPRs.
struct Slots {
  float r[TLM_EW_SLOTS];
  TLM_DEV float get(int s) const {
    switch (s) {
      case 0: return r[0];
      case 1: return r[1];
      case 2: return r[2];
      case 3: return r[3];
      case 4: return r[4];
      case 5: return r[5];
      case 6: return r[6];
      default: return r[7];
    }
  }
  TLM_DEV void set(int s, float v) {
    switch (s) {
      case 0: r[0] = v; break;
      case 1: r[1] = v; break;
      case 2: r[2] = v; break;
      case 3: r[3] = v; break;
      case 4: r[4] = v; break;
      case 5: r[5] = v; break;
      case 6: r[6] = v; break;
      default: r[7] = v; break;
    }
  }
};

__global__ __launch_bounds__(256) void ew_program(const EwArgs a) {
  for (int64_t i = blockIdx.y; i < a.rows; i += gridDim.y) {
    for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j < a.cols;
         j += (int64_t)gridDim.x * 256) {
      Slots s;
#pragma unroll
      for (int k = 0; k < TLM_EW_SLOTS; ++k) s.r[k] = 0.f;
      for (int pc = 0; pc < a.n_code; ++pc) {
        const uint32_t w = a.code[pc];
        const int op = (int)(w & 0xff), d = (int)((w >> 8) & 0xf), x = (int)((w >> 12) & 0xf),
                  y = (int)((w >> 16) & 0xf), imm = (int)((w >> 20) & 0xff);
        const float fa = s.get(x), fb = s.get(y);
        float v = 0.f;
        switch (op) {
          case TLM_EW_LOAD: {
            const int bc = a.in_bc[imm];
            const int64_t idx = bc == TLM_EW_FULL ? i * a.cols + j
                                : bc == TLM_EW_ROW ? i
                                : bc == TLM_EW_COL ? j : 0;
            v = ew_to_f32(a.in[imm], idx, a.in_dt[imm]);
            break;
          }
          case TLM_EW_CONST: v = a.cst[imm]; break;
          case TLM_EW_ADD: v = fa + fb; break;
          case TLM_EW_SUB: v = fa - fb; break;
          case TLM_EW_MUL: v = fa * fb; break;
          case TLM_EW_DIV: v = fa / fb; break;
          case TLM_EW_EXP: v = expf(fa); break;
          case TLM_EW_RSQRT: v = 1.0f / sqrtf(fa); break;
          case TLM_EW_SIGMOID: v = 1.0f / (1.0f + expf(-fa)); break;
          case TLM_EW_ROUND: v = ew_round(fa, imm); break;
          default: {  // TLM_EW_STORE: output imm <- slot x
            const int64_t idx = i * a.cols + j;
            const int dt = a.out_dt[imm];
            if (dt == TLM_F32)
              ((float*)a.out[imm])[idx] = fa;
            else
              ((uint16_t*)a.out[imm])[idx] =
                  (uint16_t)(dt == TLM_BF16 ? f32_to_bf16_bits(fa) : f32_to_f16_bits(fa));
            continue;
          }
        }
        s.set(d, v);
      }
    }
  }
}

bool ew_float(int dt) { return dt == TLM_F32 || dt == TLM_F16 || dt == TLM_BF16; }
size_t ew_esize(int dt) { return dt == TLM_F32 ? 4 : 2; }

}  // namespace

extern "C" int tlm_elementwise(const void* const* in, const int* in_dtype, const int* in_bcast,
                               int n_in, void* const* out, const int* out_dtype, int n_out,
                               const int32_t* code, int n_code, const float* consts, int n_const,
                               int64_t rows, int64_t cols, void* stream) {
  const char* fn = "tlm_elementwise";
  if (n_in < 0 || n_in > TLM_EW_MAX_IN || n_out < 1 || n_out > TLM_EW_MAX_OUT || n_code < 1 ||
      n_code > TLM_EW_MAX_CODE || n_const < 0 || n_const > TLM_EW_MAX_CONST) {
    tlm_set_error("%s: at most %d inputs, 1..%d outputs, 1..%d instructions and %d constants",
                  fn, TLM_EW_MAX_IN, TLM_EW_MAX_OUT, TLM_EW_MAX_CODE, TLM_EW_MAX_CONST);
    return TLM_EINVAL;
  }
  if ((n_in && (!in || !in_dtype || !in_bcast)) || !out || !out_dtype || !code ||
      (n_const && !consts)) {
    tlm_set_error("%s: null pointer argument", fn);
    return TLM_EINVAL;
  }
  if (rows < 0 || cols < 0 || rows > ((int64_t)1 << 40) || cols > ((int64_t)1 << 40)) {
    tlm_set_error("%s: bad shape rows=%lld cols=%lld", fn, (long long)rows, (long long)cols);
    return TLM_EINVAL;
  }
  EwArgs a = {};
  for (int k = 0; k < n_in; ++k) {
    if (!in[k] || !ew_float(in_dtype[k]) || in_bcast[k] < TLM_EW_FULL ||
        in_bcast[k] > TLM_EW_SCALAR || !tlm_aligned(in[k], ew_esize(in_dtype[k]))) {
      tlm_set_error("%s: input %d: null or misaligned pointer, dtype %d or broadcast kind %d", fn,
                    k, in_dtype[k], in_bcast[k]);
      return TLM_EINVAL;
    }
    a.in[k] = in[k];
    a.in_dt[k] = in_dtype[k];
    a.in_bc[k] = in_bcast[k];
  }
  for (int k = 0; k < n_out; ++k) {
    if (!out[k] || !ew_float(out_dtype[k]) || !tlm_aligned(out[k], ew_esize(out_dtype[k]))) {
      tlm_set_error("%s: output %d: null or misaligned pointer or dtype %d", fn, k,
                    out_dtype[k]);
      return TLM_EINVAL;
    }
    a.out[k] = out[k];
    a.out_dt[k] = out_dtype[k];
  }
  for (int pc = 0; pc < n_code; ++pc) {
    const uint32_t w = (uint32_t)code[pc];
    const int op = (int)(w & 0xff), d = (int)((w >> 8) & 0xf), x = (int)((w >> 12) & 0xf),
              y = (int)((w >> 16) & 0xf), imm = (int)((w >> 20) & 0xff);
    const bool slots_ok = d < TLM_EW_SLOTS && x < TLM_EW_SLOTS && y < TLM_EW_SLOTS;
    bool ok = slots_ok && op <= TLM_EW_STORE && (w >> 28) == 0;
    if (op == TLM_EW_LOAD) ok = ok && imm < n_in;
    if (op == TLM_EW_CONST) ok = ok && imm < n_const;
    if (op == TLM_EW_STORE) ok = ok && imm < n_out;
    if (op == TLM_EW_ROUND) ok = ok && (imm == TLM_F16 || imm == TLM_BF16 || imm == TLM_F32);
    if (!ok) {
      tlm_set_error("%s: instruction %d (0x%08x) is malformed", fn, pc, w);
      return TLM_EINVAL;
    }
    a.code[pc] = w;
  }
  for (int k = 0; k < n_const; ++k) a.cst[k] = consts[k];
  a.n_code = n_code;
  a.rows = rows;
  a.cols = cols;
  if (rows == 0 || cols == 0) return TLM_OK;
  const unsigned gx = (unsigned)std::min<int64_t>((cols + 255) / 256, 64);
  const unsigned gy = (unsigned)std::min<int64_t>(rows, 65535);
  ew_program<<<dim3(gx, gy), 256, 0, (hipStream_t)stream>>>(a);
  TLM_LAUNCH_CHECK("tlm_elementwise");
  return TLM_OK;
}
