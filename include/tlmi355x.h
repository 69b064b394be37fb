/*
 * tlmi355x.h — C ABI of libtlmi355x.so, the gfx950 (MI355X) kernels that sit behind
 * `tilelang.compile(..., target="mi355x")`.
 *
 * The reference crosses its process/device boundary through one generated entry point,
 *   extern "C" int tilelang_tpu_run(void** args)
 * (reference: src/tl_templates/tpu/main_template.cpp:39, bound by ctypes at
 *  tilelang/jit/adapter/cython/adapter.py:214-216 with argtypes=[POINTER(c_void_p)],
 *  restype=c_int), which is regenerated per kernel from templates
 * (tilelang/jit/adapter/wrapper.py:617-834). This library replaces that per-kernel
 * codegen with one fixed entry point per operator family. The Python adapter binds
 * these with ctypes exactly as the reference binds tilelang_tpu_run.
 *
 * Conventions (all entry points):
 *  - every pointer is a DEVICE pointer owned by the caller (torch allocates); the
 *    library allocates nothing on the hot path (MLA takes its workspace from the caller, or
 *    uses the library-owned scratch array of tlm_mla_decode_noalloc);
 *  - tensors are dense, row-major (C-contiguous) unless a stride argument says otherwise;
 *  - return 0 on success or a negative TLM_E* code; the message is available from
 *    tlm_last_error() (thread-local). Nothing aborts or prints;
 *  - argument validation runs BEFORE any HIP call, so every error path is testable on a
 *    host without a GPU;
 *  - `stream` is a hipStream_t (torch.cuda.current_stream().cuda_stream), NULL = default;
 *  - calls are reentrant; per-device state is initialised once (std::call_once).
 */
#ifndef TLMI355X_H
#define TLMI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. Mirrors the reference's dtype table for generated wrappers
 * (tilelang/jit/adapter/wrapper.py:622-648) restricted to what the kernels take. */
enum tlm_dtype {
  TLM_F16 = 0,
  TLM_BF16 = 1,
  TLM_F32 = 2,
  TLM_F8E4M3 = 3, /* OCP e4m3fn (gfx950 native), not the FNUZ variant of gfx942 */
  TLM_I32 = 4,
  TLM_F8E5M2 = 5, /* OCP e5m2 */
  TLM_U32 = 6,
};

/* Row reductions of tlm_row_reduce (ppl_reduce_max / ppl_reduce_sum). */
enum tlm_reduce_op {
  TLM_REDUCE_MAX = 0,
  TLM_REDUCE_SUM = 1,
};

/* Error codes. The reference returns -1 (init), -2 (module load), 1 (launch)
 * (main_template.cpp:15-31, 64-67); here every failure is negative. */
enum tlm_status {
  TLM_OK = 0,
  TLM_EINVAL = -1,       /* null/misaligned pointer, bad size or dtype */
  TLM_EUNSUPPORTED = -2, /* valid request that no kernel here implements */
  TLM_EHIP = -3,         /* a HIP runtime call failed (message names it) */
  TLM_EWORKSPACE = -4,   /* caller workspace too small */
};

/* Library version (major*10000 + minor*100 + patch). No reference counterpart. */
int tlm_version(void);

/* Select and initialise `device` (hipSetDevice + property query, once per device).
 * Replaces init() of main_template.cpp:14-32 (tpuRtInit/tpuRtSetDevice). */
int tlm_init(int device);

/* Message for the last failing call on this thread ("" if none). Replaces the
 * GPU-side get_last_error() convention (wrapper.py:22-42). */
const char* tlm_last_error(void);

/* Number of compute units of the current device (0 if unknown). */
int tlm_num_cus(void);

/* RMSNorm over the last dim: y[r,:] = cast(x[r,:] * rsqrt(mean_fp32(x[r,:]^2) + eps) * w).
 * Reference program: tpu_demo/rms_norm/rms_norm_fp16.py:9-35 (no weight, eps 1e-12);
 * oracle rms_norm_fp16.py:51-54. `w` may be NULL (reference behaviour). dtype: F16 | BF16 |
 * F32 (rmsnorm_fp32.py: the same expression on fp32 tiles, stored without rounding). The
 * split-K programs (rmsnorm_splitk_{fp16,bf16,fp32}.py:9-47) compute the same result. */
int tlm_rmsnorm(const void* x, const void* w, void* y, int64_t rows, int64_t cols, float eps,
                int dtype, void* stream);

/* SwiGLU: out = cast(up * gate / (1 + exp(-gate))) in fp32.
 * Reference program tpu_demo/tpu_test_swiglu_bf16.py:5-54 (param order gate, up, out),
 * oracle :68 (b * F.silu(a)). dtype: BF16 | F16 | F32 (tpu_test_swiglu_fp32.py: fp32 out, no
 * rounding). n = number of elements. */
int tlm_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream);

/* Interleaved RoPE on x[tokens, heads, dim] with tables cos/sin[tokens, dim] shared by all
 * heads (pairs (2i, 2i+1) rotate by the angle stored at cos[t,2i] / sin[t,2i]):
 *   out[2i]   = x[2i]*c - x[2i+1]*s,   out[2i+1] = x[2i+1]*c + x[2i]*s   (fp32, one rounding).
 * Reference program tpu_demo/tpu_test_rope_bf16.py:5-51 (ppl_rope_add), oracle :76-92.
 * The reference's [C, W] program is the case heads == 1. `k`/`k_out` may be NULL; when
 * given, k[tokens, heads_k, dim] is rotated in the same launch. dtype: BF16 | F16 | F32
 * (tpu_test_rope_fp16.py, tpu_test_rope_fp32.py, tpu_test_rope.py). */
int tlm_rope(const void* q, const void* k, const void* cos_t, const void* sin_t, void* q_out,
             void* k_out, int64_t tokens, int64_t heads_q, int64_t heads_k, int64_t dim, int dtype,
             void* stream);

/* GEMM: C[M,N] = A[M,K] * B (fp32 accumulation, one rounding to out_dtype).
 * trans_b == 0: B is [K,N] row-major (reference ppl_gemm transpose_B=False,
 *   tpu_demo/matmul/tpu_test_matmul_fp16.py:9-31, src/target/codegen_ppl.cc:1244-1279).
 * trans_b == 1: B is [N,K] row-major (ppl_gemm transpose_B=True).
 * in_dtype: F16 | BF16; out_dtype: F16 | BF16 | F32. The fp32 program
 * (tpu_demo/matmul/tpu_test_matmul_fp32.py:9-31) copies its fp32 A/B tiles to fp16 before
 * ppl_gemm: tlm_cast to F16, then this with out_dtype F32.
 * M <= 16 with trans_b == 0 (and with trans_b == 1 when the output has few 64-column strips)
 * splits K over several workgroups whose partial tiles meet in a library-owned device workspace (16 MB per GPU, 4 slots): each stream owns one slot, so calls
 * on one stream are ordered and calls that overlap use different slots; further streams take an
 * unsplit kernel. A HIP graph keeps the slot of the stream it was captured on, so its replays
 * must not overlap each other or other work of that stream. Slots are keyed by the stream handle:
 * a stream created after another is destroyed can get the same handle and inherits its slot, so
 * a stream is destroyed only once its calls have finished. The result does not depend on the
 * split's timing: a stream's calls are bitwise reproducible (the unsplit kernel of a stream
 * without a slot sums in another order, so its last bits can differ from the split kernel's). */
int tlm_gemm(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int in_dtype,
             int out_dtype, int trans_b, void* stream);

/* FP8 GEMM: C[M,N] = A[M,K] * B^T with B [N,K] row-major (trans_b == 1; trans_b == 0 takes B
 * [K,N] through a per-output fallback), fp32 accumulation, one rounding to out_dtype.
 * Reference: examples/gemm_fp8/example_tilelang_gemm_fp8.py:17-37 (T.gemm transpose_B=True,
 * fp8 C; oracle (a.half() @ b.half().T).to(fp8), :46-55) and example_tilelang_gemm_fp8_2xAcc.py
 * (fp32 C). in_dtype: F8E4M3 | F8E5M2 (OCP); out_dtype: F32 | F16 | BF16 | in_dtype (round to
 * nearest even without saturation, as torch's cast). */
int tlm_gemm_fp8(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                 int in_dtype, int out_dtype, int trans_b, void* stream);

/* Elementwise sigmoid y = 1 / (1 + exp(-x)) in fp32, one rounding for 16-bit y.
 * Reference: tpu_demo/tpu_test_sigmoid_fp32.py:6-31 (T.ppl_sigmoid, fp32; customize.py:343-350),
 * checked against torch.sigmoid (:48-60). dtype: F32 | F16 | BF16; n elements. */
int tlm_sigmoid(const void* x, void* y, int64_t n, int dtype, void* stream);

/* Row gather out[i, :] = param[index[i], :] (row_bytes bytes per row; any element type).
 * Reference: tpu_demo/tpu_test_gather_fp32.py:8-18, T.ppl_gather (customize.py:352-356) ->
 * tpu_gdma_h_gather_S2S (src/target/codegen_ppl.cc:1849-1877), param_h = param_rows, uint32
 * indices. An index >= param_rows writes a zero row. */
int tlm_gather_rows(const void* param, int64_t param_rows, int64_t row_bytes,
                    const uint32_t* index, int64_t n_index, void* out, void* stream);

/* Sort of a vector with its indices; the first k entries are the top k.
 * Reference: tpu_demo/tpu_test_topk_fp32.py:6-18, T.ppl_topk (customize.py:358-362) ->
 * tpu_hau_sort_natural_index(dst, dst_idx, src, length, K, descended) (codegen_ppl.cc:1878-1907),
 * which writes `length` sorted entries. Order: by value (descending when `descending` != 0),
 * ties by index, every NaN above +inf, -0.0 equal to +0.0 (torch.sort(stable=True)).
 * dtype: F32 | I32 | U32; length <= 16384 (one workgroup, LDS bitonic sort). */
int tlm_topk(const void* src, int64_t length, int64_t k, int descending, int dtype,
             void* out_values, int32_t* out_indices, void* stream);

/* Row reduction y[r] = max_c / sum_c x[r, c] (op TLM_REDUCE_MAX | TLM_REDUCE_SUM).
 * Reference: tpu_demo/tpu_test_reduce_max.py, tpu_test_reduce_sum.py (X [M, N] -> Y [M, 1],
 * T.ppl_reduce_max / ppl_reduce_sum, customize.py:476-573). Sum in fp32, rounded once; max
 * propagates NaN. in_dtype, out_dtype: F32 | F16 | BF16. */
int tlm_row_reduce(const void* x, void* y, int64_t rows, int64_t cols, int op, int in_dtype,
                   int out_dtype, void* stream);

/* Element-type conversion of n contiguous values, the cast of a ppl_copy between tiles of
 * different dtypes (src/target/codegen_ppl.cc:1138-1152): F32 -> F16 | BF16 rounds to nearest
 * even, F16 | BF16 -> F32 is exact. Used for the fp32 demo programs whose matrix operands are
 * fp16 tiles (tpu_test_matmul_fp32.py:22-28, flashattn/tpu_test_flashattn_fp32.py:28-55). */
int tlm_cast(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, void* stream);

/* FlashAttention forward, BSHD layout: q,k,v,o [B, S, H, D]; softmax in fp32 with scale
 * sm_scale; P rounded to the input dtype before P*V; causal masks key j > query i.
 * Reference: tpu_demo/flashattn/tpu_test_flashattn_bf16.py:14-135 (oracle :171-182),
 * element mask per examples/flash_attention/example_mha_fwd_bshd.py:50-53.
 * dtype: BF16 | F16 (q, k, v and o). D: any multiple of 8 up to 256 (tiled MFMA kernels for
 * 128 and 64; other head dims, such as the demo programs' dim 8, run a per-query kernel). */
int tlm_flash_attn_fwd(const void* q, const void* k, const void* v, void* o, int64_t B, int64_t S,
                       int64_t H, int64_t D, int causal, float sm_scale, int dtype, void* stream);

/* General form of tlm_flash_attn_fwd.
 *   H_kv: K and V are [B, S, H_kv, D] and query head h attends with K/V head h / (H / H_kv)
 *         (grouped-query attention, examples/flash_attention/example_gqa_fwd_bshd.py:92-100:
 *         K[bz, .., by // groups, :]); H_kv == H is multi-head attention. H % H_kv == 0.
 *   out_dtype: in_dtype or F32. The fp32 demo program
 *         (tpu_demo/flashattn/tpu_test_flashattn_fp32.py:14-135) multiplies fp16 copies of its
 *         fp32 Q/K/V tiles and of P but keeps acc_o and the output in fp32: tlm_cast Q, K, V to
 *         F16, then this with in_dtype F16, out_dtype F32.
 *   in_dtype F32 (out_dtype F32, D a multiple of 4): all-fp32 attention with no 16-bit
 *         rounding, the program tpu_demo/ppl/flashattn/fa_fp32.py:10-125 (fp32 tiles into
 *         ppl_gemm, fp32 P); a per-query correctness kernel, not a tuned one. */
int tlm_flash_attn_fwd_ex(const void* q, const void* k, const void* v, void* o, int64_t B,
                          int64_t S, int64_t H, int64_t H_kv, int64_t D, int causal,
                          float sm_scale, int in_dtype, int out_dtype, void* stream);

/* Variable-length FlashAttention forward on unpadded sequences.
 * Reference: examples/flash_attention/example_mha_fwd_varlen.py:222-358 (params Q_unpad,
 * K_unpad, V_unpad, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, Output_unpad, :239-247).
 *   q, o [total_q, H, D]; k, v [total_k, H_kv, D]; sequence b holds query rows
 *   cu_seqlens_q[b] .. cu_seqlens_q[b + 1] - 1 and key rows cu_seqlens_k[b] .. [b + 1] - 1
 *   (int32 [B + 1] device arrays, :267-276). Query i of a sequence attends to every key of its
 *   sequence (the example's mask, :304-307); causal (extension) keeps key j <= i + nk - nq, the
 *   bottom-right alignment of the file's construct_local_mask (:156-157). A query row with no
 *   visible key gets zeros.
 *   max_seqlen_q sizes the grid, as the example's T.ceildiv(max_seqlen_q, block_M) (:249):
 *   queries at positions >= max_seqlen_q are not computed and their rows of o are left as
 *   they were. A sequence whose rows fall outside [0, total_q) / [0, total_k) is skipped (o
 *   untouched), so device-side offsets cannot address memory outside the tensors.
 *   Other arguments as tlm_flash_attn_fwd_ex. */
int tlm_flash_attn_varlen_fwd(const void* q, const void* k, const void* v, void* o,
                              const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                              int64_t B, int64_t max_seqlen_q, int64_t total_q, int64_t total_k,
                              int64_t H, int64_t H_kv, int64_t D, int causal, float sm_scale,
                              int in_dtype, int out_dtype, void* stream);

/* FlashAttention forward on head-major tensors.
 * Reference: examples/flash_attention/example_mha_fwd_bhsd.py:30-158 (main(Q, K, V, Output),
 * :115-119; q_shape [batch, heads, seq_q, dim], kv_shape [batch, heads, seq_kv, dim], :32-33).
 *   q, o [B, H, S_q, D]; k, v [B, H_kv, S_kv, D], H % H_kv == 0 (query head h reads K/V head
 *   h / (H / H_kv)). S_q and S_kv may differ. Causal keeps key j <= i + S_kv - S_q for query i,
 *   the example's mask q_idx = bx * block_M + i + past_len, past_len = seq_kv - seq_q (:50-55);
 *   a query row with no visible key gets zeros. Other arguments as tlm_flash_attn_fwd_ex. */
int tlm_flash_attn_bhsd_fwd(const void* q, const void* k, const void* v, void* o, int64_t B,
                            int64_t H, int64_t H_kv, int64_t S_q, int64_t S_kv, int64_t D,
                            int causal, float sm_scale, int in_dtype, int out_dtype,
                            void* stream);

/* Split-KV inference attention: the program's partial outputs and their combine.
 * Reference: examples/flash_attention/example_mha_inference.py:10-203 (flash_attn_split :98-160,
 * combine :162-203, main(Q, K, V, glse, Output_partial, Output) :187-203).
 *   q, o [B, S_q, H, D]; k, v [B, S_kv, H_kv, D]; glse [B, H, num_split, S_q];
 *   o_partial [B, S_q, H, num_split, D]; all of `dtype` (F16 | BF16), dense.
 *   Split s covers keys [s P, (s + 1) P), P = S_kv / num_split (S_kv must be a multiple of
 *   num_split, 1 <= num_split <= 16). o_partial[b, q, h, s] = the split's normalised output and
 *   glse[b, h, s, q] = log2(l) + m, the split's log2 sum-exp of the scaled scores (exp2 domain,
 *   scale = sm_scale * log2 e), both rounded to `dtype`; o = the program's combine of those
 *   stored values. Non-causal (the program's causal form has no split offset).
 *   ws: caller workspace of at least tlm_flash_attn_splitkv_workspace_bytes() bytes (16-byte
 *   aligned): the splits are cut into finer key parts so the launch fills every CU, and the parts
 *   are merged exactly (fp32) before the per-split rounding. */
size_t tlm_flash_attn_splitkv_workspace_bytes(int64_t B, int64_t S_q, int64_t S_kv, int64_t H,
                                             int64_t D, int num_split);
int tlm_flash_attn_splitkv_fwd(const void* q, const void* k, const void* v, void* glse,
                               void* o_partial, void* o, void* ws, size_t ws_bytes, int64_t B,
                               int64_t S_q, int64_t S_kv, int64_t H, int64_t H_kv, int64_t D,
                               int num_split, float sm_scale, int dtype, void* stream);

/* Elementwise tile programs: the stand-alone T.ppl_* elementwise programs of the TPU demos
 * (tpu_demo/ppl/test/exp.py:6-16, mul_N_1.py:9-22, elementwise_c.py:9-22,
 * tpu_demo/ppl/elementwise_add_kernel/elementwise_add.py:9-35; ops language/customize.py:238-339,
 * 377-472), compiled by the recogniser into a register program run for every element (i, j) of
 * the [rows, cols] output domain (replaces the PPL codegen of those programs).
 *   in[k]   input k (in_dtype F32 | F16 | BF16), read at i * cols + j (TLM_EW_FULL), i
 *           (TLM_EW_ROW: an [rows, 1] tensor broadcast along the row, the (M, 1) operand of
 *           ppl_add / ppl_mul, codegen_ppl.cc:874-883), j (TLM_EW_COL) or 0 (TLM_EW_SCALAR);
 *   out[k]  output k (out_dtype), written at i * cols + j, rounded to nearest even;
 *   code    n_code instruction words: op | dst << 8 | a << 12 | b << 16 | imm << 20, slots
 *           0..TLM_EW_SLOTS-1 holding fp32 values (initially 0). LOAD dst <- in[imm];
 *           CONST dst <- consts[imm]; ADD / SUB / MUL / DIV dst <- a op b; EXP dst <- e^a;
 *           RSQRT dst <- 1 / sqrt(a); SIGMOID dst <- 1 / (1 + e^-a); ROUND dst <- a rounded to
 *           dtype imm (F16 / BF16 / F32: the value a 16-bit tile holds); STORE out[imm] <- a.
 * Outputs may alias inputs only element for element (the in-place exp.py). */
#define TLM_EW_MAX_IN 8
#define TLM_EW_MAX_OUT 4
#define TLM_EW_MAX_CODE 64
#define TLM_EW_MAX_CONST 16
#define TLM_EW_SLOTS 8
enum tlm_ew_op {
  TLM_EW_LOAD = 0,
  TLM_EW_CONST = 1,
  TLM_EW_ADD = 2,
  TLM_EW_SUB = 3,
  TLM_EW_MUL = 4,
  TLM_EW_DIV = 5,
  TLM_EW_EXP = 6,
  TLM_EW_RSQRT = 7,
  TLM_EW_SIGMOID = 8,
  TLM_EW_ROUND = 9,
  TLM_EW_STORE = 10,
};
enum tlm_ew_bcast {
  TLM_EW_FULL = 0,
  TLM_EW_ROW = 1,
  TLM_EW_COL = 2,
  TLM_EW_SCALAR = 3,
};
int tlm_elementwise(const void* const* in, const int* in_dtype, const int* in_bcast, int n_in,
                    void* const* out, const int* out_dtype, int n_out, const int32_t* code,
                    int n_code, const float* consts, int n_const, int64_t rows, int64_t cols,
                    void* stream);

/* MLA paged decode (one query token per sequence, one shared latent KV head).
 * Reference: examples/deepseek_mla/example_mla_decode_paged.py:10-256 (split kernel :100-183,
 * LSE combine :186-221, params :224-256), torch oracle :259-308.
 *   q      [B, Hq, q_stride] (q_stride >= dqk): q[..., :dv] is the latent part, q[..., dv:dqk]
 *          the rope part; q_pe may point elsewhere (q_pe_stride) to take the reference's
 *          separate Q / Q_pe tensors; pass q_pe = q + dv elements for a fused [.., 576] tensor.
 *   kv     token rows of the paged cache; row t at kv + t*kv_stride holds the dv latent values,
 *   k_pe   row t at k_pe + t*kpe_stride holds the dpe rope values (same convention as q_pe).
 *   kv_rows number of token rows in the cache pool; a row index outside [0, kv_rows) produced by
 *          a corrupt block table is read as zeros instead of faulting.
 *   block_table int32 [B, max_pages]: token j of sequence b lives in row
 *          block_table[b, j / page] * page + j % page   (example_mla_decode_paged.py:62-63).
 *   seqlens int32 [B], each in [0, max_pages*page] (larger values are clamped to
 *          max_pages*page; a zero-length sequence gets a zero output row).
 *   o      [B, Hq, dv] out dtype (F16 | BF16).
 * kv_dtype: F8E4M3 (value = e4m3 decode of the byte times *kv_scale, a DEVICE fp32 scalar so
 *   that no host sync is needed; NULL means 1) | F16 | BF16 (kv_scale may be NULL).
 * q_dtype: BF16 | F16. The softmax uses sm_scale (natural-log domain).
 * num_split >= 1 KV splits per sequence, combined by an LSE pass through `ws`. With fp8 KV, page
 *   a multiple of 64 and Hq a multiple of 64 the decode runs on the fp8 matrix cores with the
 *   sequences' tiles balanced over B*num_split/(Hq/64) ranges (num_split then only sets the
 *   parallelism); other cases use one workgroup per (sequence, split, 64 heads).
 * dv = 512, dpe = 64, Hq a multiple of 64 and 16-byte aligned Q / KV rows take those
 *   matrix-core kernels; any other dv <= 1024, dpe <= 256, Hq <= 4096 (e.g. the TPU program
 *   tpu_demo/ppl/deepseek_mla/mla_decode.py at dim 32 + rope 4 over 8 heads) runs a generic
 *   per-(sequence, head) kernel that needs no workspace.
 * A non-paged cache [B, S, 1, d] (examples/deepseek_mla/example_mla_decode.py) is the paged
 *   layout with page = S, max_pages = 1 and block_table[b, 0] = b.
 * ws must hold tlm_mla_workspace_bytes(...) bytes (device memory, caller-owned; the largest of
 *   the paths' layouts, the split programs' fp8 path of tlm_mla_decode_ex included). */
int tlm_mla_decode(const void* q, const void* q_pe, int64_t q_stride, int64_t q_pe_stride,
                   const void* kv, const void* k_pe, int64_t kv_stride, int64_t kpe_stride,
                   int64_t kv_rows, const int32_t* block_table, const int32_t* seqlens, void* o,
                   void* ws,
                   size_t ws_bytes, int64_t B, int64_t Hq, int64_t dv, int64_t dpe, int64_t page,
                   int64_t max_pages, int num_split, float sm_scale, const float* kv_scale,
                   int q_dtype, int kv_dtype, int o_dtype, void* stream);

/* tlm_mla_decode for the split programs that keep their partials: the split kernel of
 * examples/deepseek_mla/example_mla_decode_paged.py:100-183 writes glse [b, h, s] and
 * Output_partial [b, h, s, :] (:182-184) and its combine (:186-221) reads them back; the non-paged
 * example_mla_decode.py split form does the same.
 *   glse [B, Hq, num_split] and o_partial [B, Hq, num_split, dv], dense, of p_dtype (F16 | BF16 |
 *   F32, the last stored without rounding):
 *   split s of a sequence holds its blocks of part_block tokens dealt out so that the first
 *   (blocks % num_split) splits take one extra (the program's block_N; :140-144). o_partial
 *   receives the split's normalised output (times kv_scale for fp8 KV) and glse its log2
 *   sum-exp of the scaled scores (exp2 domain), both rounded to p_dtype; o is the combine of the
 *   stored values. A split without tokens stores -inf and zeros (the reference divides 0 by 0
 *   there). dv must be a multiple of 4. With glse and o_partial both NULL this is
 *   tlm_mla_decode. With fp8 KV, part_block 64, Hq a multiple of 128, dv 512 / dpe 64 and a
 *   workspace of tlm_mla_workspace_bytes(...) the program's splits run as segments of their
 *   sequences on the balanced 128-head fp8 decode (glse then sums the e4m3-rounded P that
 *   weighs the split's output: within ~0.1 of the exact log2 sum-exp); other requests run the
 *   program's partition on the split kernels. Other arguments as tlm_mla_decode. */
int tlm_mla_decode_ex(const void* q, const void* q_pe, int64_t q_stride, int64_t q_pe_stride,
                      const void* kv, const void* k_pe, int64_t kv_stride, int64_t kpe_stride,
                      int64_t kv_rows, const int32_t* block_table, const int32_t* seqlens,
                      void* o, void* ws, size_t ws_bytes, int64_t B, int64_t Hq, int64_t dv,
                      int64_t dpe, int64_t page, int64_t max_pages, int num_split,
                      float sm_scale, const float* kv_scale, int q_dtype, int kv_dtype,
                      int o_dtype, void* glse, void* o_partial, int64_t part_block, int p_dtype,
                      void* stream);

/* Workspace bytes that tlm_mla_decode and tlm_mla_decode_ex need for (B, Hq, dv, num_split). */
size_t tlm_mla_workspace_bytes(int64_t B, int64_t Hq, int64_t dv, int num_split);

/* Bytes of the library-owned scratch of tlm_mla_decode_noalloc (per GPU). */
#define TLM_MLA_SCRATCH_BYTES ((size_t)128 << 20)

/* tlm_mla_decode without a caller workspace and without any allocation: the kernels' scratch
 * (tile prefix, Q terms, partial outputs and log-sum-exps) lives in a library-owned device array
 * of TLM_MLA_SCRATCH_BYTES, one per GPU, held from the library's first use on that GPU until the
 * process ends. No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). Same
 * arguments, validation and results as tlm_mla_decode (ws / ws_bytes dropped). Returns
 * TLM_EWORKSPACE, before any HIP call, when the path taken needs more scratch than
 * TLM_MLA_SCRATCH_BYTES (the FP8 config B 64, Hq 128 with num_split <= 4 fits). Every call on a
 * GPU shares that GPU's array and nothing in it has to start zeroed; calls that overlap in time on
 * one GPU (several streams or host threads) race on it and must be serialised by the caller. */
int tlm_mla_decode_noalloc(const void* q, const void* q_pe, int64_t q_stride, int64_t q_pe_stride,
                           const void* kv, const void* k_pe, int64_t kv_stride, int64_t kpe_stride,
                           int64_t kv_rows, const int32_t* block_table, const int32_t* seqlens,
                           void* o, int64_t B, int64_t Hq, int64_t dv, int64_t dpe, int64_t page,
                           int64_t max_pages, int num_split, float sm_scale,
                           const float* kv_scale, int q_dtype, int kv_dtype, int o_dtype,
                           void* stream);

/* TLM_MLA_SCRATCH_BYTES, for bindings that cannot read the macro. */
size_t tlm_mla_scratch_bytes(void);

/* Integer-path check: out[i, :] = kv_bytes[row(i), :] for every token i of every sequence,
 * rows resolved through the block table exactly as tlm_mla_decode does; tokens of sequence b
 * are written at out + (cu_seqlens[b] + j) * row_bytes with cu_seqlens the exclusive prefix
 * sum of seqlens (computed on the host by the caller and passed in). Rows outside [0, kv_rows)
 * are written as zeros. Bit-exact by contract. */
int tlm_paged_gather(const void* kv_bytes, int64_t row_bytes, int64_t kv_rows,
                     const int32_t* block_table, const int32_t* seqlens, const int64_t* cu_seqlens,
                     void* out, int64_t B, int64_t page, int64_t max_pages, void* stream);

/* Paged KV-cache append with FP8 (OCP e4m3) quantisation, the step that fills the cache
 * tlm_mla_decode reads. For every sequence b and each of its count[b] new tokens j
 * (0 <= j < min(count[b], T)), at position p = start[b] + j:
 *   kv[row(p)] = e4m3(clamp(x[b, j, :] / *scale, -448, 448))   (NaN stays NaN)
 * with row(p) = block_table[b, p / page] * page + p % page, the decode's page addressing
 * (examples/deepseek_mla/example_mla_decode_paged.py:62-63; table layout :26). No reference
 * program implements this step; the quantisation equals the MLA config's cache construction
 * (x / scale).to(float8_e4m3fn) for in-range values and saturates beyond +-448.
 *   x      [B, T, D] rows of D elements (x_dtype BF16 | F16) at x + b*x_batch_stride +
 *          j*x_row_stride (elements; strides and D multiples of 8, x 16-byte aligned)
 *   kv     fp8 pool rows of kv_stride bytes, kv_rows rows (8-byte aligned)
 *   scale  device pointer to the fp32 dequantisation scale (value = code * scale)
 * Positions beyond the table and rows outside [0, kv_rows) are skipped (nothing written). */
int tlm_kv_append_fp8(const void* x, int64_t x_batch_stride, int64_t x_row_stride, int x_dtype,
                      const int32_t* start, const int32_t* count, const int32_t* block_table,
                      int64_t max_pages, int64_t page, void* kv, int64_t kv_stride,
                      int64_t kv_rows, int64_t B, int64_t T, int64_t D, const float* scale,
                      void* stream);

#ifdef __cplusplus
}
#endif
#endif /* TLMI355X_H */
