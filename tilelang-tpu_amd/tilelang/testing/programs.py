"""Kernel programs for the six families, written with ``tilelang.language``.

They restate the op sequences of the reference's demo programs (the recogniser keys on those
sequences, so a reference script compiles unchanged):
  rms_norm   tpu_demo/rms_norm/rms_norm_fp16.py:9-35   (+ optional weight parameter)
  matmul     tpu_demo/matmul/tpu_test_matmul_fp16.py:9-31
  rope       tpu_demo/tpu_test_rope_bf16.py:5-51        (rope_qk: q and k with shared tables)
  swi_glu    tpu_demo/tpu_test_swiglu_bf16.py:5-54
  flashattn  tpu_demo/flashattn/tpu_test_flashattn_bf16.py:14-135
  mla_decode examples/deepseek_mla/example_mla_decode_paged.py:10-256 (+ fp8 KV with a scale)
"""
import tilelang.language as T


def rms_norm(M, N, blk_m, dtype="float16", eps=1e-12, with_weight=False):
    """rms_norm_fp16.py:9-35 (bf16 twin); dtype float32 gives rmsnorm_fp32.py, which squares and
    scales the fp32 tile directly (no cast copies)."""
    rN = 1.0 / N
    f32 = dtype == "float32"

    def body(A, W, B):
        with T.Kernel(T.ceildiv(M, blk_m), is_cpu=True) as (bx,):
            x_tile = T.alloc_shared((blk_m, N), dtype)
            x32 = x_tile if f32 else T.alloc_shared((blk_m, N), "float32")
            sq = T.alloc_shared((blk_m, N), "float32")
            ssum = T.alloc_shared((blk_m, 1), "float32")
            T.ppl_copy(A[bx * blk_m, 0], x_tile)
            if not f32:
                T.ppl_copy(x_tile, x32)
            T.ppl_mul(sq, x32, x32)
            T.ppl_reduce_sum(sq, ssum, dim=1)
            T.ppl_mul_C(ssum, ssum, T.float32(rN))
            T.ppl_add_C(ssum, ssum, T.float32(eps))
            T.ppl_rsqrt(ssum, ssum)
            T.ppl_mul(x32, x32, ssum)
            if W is not None:
                w_tile = T.alloc_shared((1, N), dtype)
                w32 = w_tile if f32 else T.alloc_shared((1, N), "float32")
                T.ppl_copy(W[0], w_tile)
                if not f32:
                    T.ppl_copy(w_tile, w32)
                T.ppl_mul(x32, x32, w32)
            if not f32:
                T.ppl_copy(x32, x_tile)
            T.ppl_copy(x_tile, B[bx * blk_m, 0])

    if with_weight:

        @T.prim_func
        def rmsnorm_w(A: T.Tensor((M, N), dtype), W: T.Tensor((N,), dtype),
                      B: T.Tensor((M, N), dtype)):
            body(A, W, B)

        return rmsnorm_w

    @T.prim_func
    def rmsnorm(A: T.Tensor((M, N), dtype), B: T.Tensor((M, N), dtype)):
        body(A, None, B)

    return rmsnorm


def rms_norm_splitk(M, N, blk_m, blk_k, dtype="float16", eps=1e-12):
    """rmsnorm_splitk_fp16.py:9-47 (bf16 / fp32 twins): the row sum of squares accumulated over
    column blocks of blk_k, then a second pass over the blocks scales them."""
    rN = 1.0 / N
    f32 = dtype == "float32"

    @T.prim_func
    def rmsnorm_splitk(A: T.Tensor((M, N), dtype), B: T.Tensor((M, N), dtype)):
        with T.Kernel(T.ceildiv(M, blk_m), is_cpu=True) as (bx,):
            a_s = T.alloc_shared((blk_m, blk_k), dtype)
            a32 = a_s if f32 else T.alloc_shared((blk_m, blk_k), "float32")
            sq = T.alloc_shared((blk_m, blk_k), "float32")
            powsum = T.alloc_shared((blk_m, 1), "float32")
            tmp = T.alloc_shared((blk_m, 1), "float32")
            T.ppl_fill(powsum, T.float32(0.0))
            nk = T.ceildiv(N, blk_k)
            for k in T.Pipelined(nk, num_stages=0):
                T.ppl_copy(A[bx * blk_m, k * blk_k], a_s)
                if not f32:
                    T.ppl_copy(a_s, a32)
                T.ppl_mul(sq, a32, a32)
                T.ppl_reduce_sum(sq, tmp, dim=1)
                T.ppl_add(powsum, powsum, tmp)
            T.ppl_mul_C(powsum, powsum, T.float32(rN))
            T.ppl_add_C(powsum, powsum, T.float32(eps))
            T.ppl_rsqrt(powsum, powsum)
            for k in T.Pipelined(nk, num_stages=0):
                kb = nk - 1 - k
                T.ppl_copy(A[bx * blk_m, kb * blk_k], a_s)
                if not f32:
                    T.ppl_copy(a_s, a32)
                T.ppl_mul(a32, a32, powsum)
                if not f32:
                    T.ppl_copy(a32, a_s)
                T.ppl_copy(a_s, B[bx * blk_m, kb * blk_k])

    return rmsnorm_splitk


def matmul(M, N, K, block_M, block_N, block_K, dtype="float16", out_dtype="float16",
           trans_b=False, operand_dtype=None):
    """tpu_test_matmul_fp16.py:9-31 (bf16 / fp32-out twins); dtype float32 with operand_dtype
    float16 gives tpu_test_matmul_fp32.py (fp32 tiles copied to fp16 tiles before ppl_gemm)."""
    b_shape = (N, K) if trans_b else (K, N)
    b_tile = (block_N, block_K) if trans_b else (block_K, block_N)
    op_dt = operand_dtype or dtype

    @T.prim_func
    def gemm(A: T.Tensor((M, K), dtype), B: T.Tensor(b_shape, dtype),
             C: T.Tensor((M, N), out_dtype)):
        with T.Kernel(T.ceildiv(N, block_N), T.ceildiv(M, block_M), is_cpu=True) as (bx, by):
            a_s = T.alloc_shared((block_M, block_K), dtype)
            b_s = T.alloc_shared(b_tile, dtype)
            a_op = a_s if op_dt == dtype else T.alloc_shared((block_M, block_K), op_dt)
            b_op = b_s if op_dt == dtype else T.alloc_shared(b_tile, op_dt)
            acc = T.alloc_shared((block_M, block_N), "float32")
            c_s = T.alloc_shared((block_M, block_N), out_dtype)
            T.ppl_fill(acc, T.float32(0))
            for k in T.Pipelined(T.ceildiv(K, block_K), num_stages=2):
                T.ppl_copy(A[by * block_M, k * block_K], a_s)
                if trans_b:
                    T.ppl_copy(B[bx * block_N, k * block_K], b_s)
                else:
                    T.ppl_copy(B[k * block_K, bx * block_N], b_s)
                if op_dt != dtype:
                    T.ppl_copy(a_s, a_op)
                    T.ppl_copy(b_s, b_op)
                T.ppl_gemm(a_op, b_op, acc, transpose_B=trans_b)
            T.ppl_copy(acc, c_s)
            T.ppl_copy(c_s, C[by * block_M, bx * block_N])

    return gemm


def matmul_fp8(M, N, K, block_M=128, block_N=128, block_K=64, dtype="e4m3_float8",
               out_dtype=None, two_acc=False):
    """examples/gemm_fp8/example_tilelang_gemm_fp8.py:17-37 (C in the fp8 input type) and, with
    two_acc, example_tilelang_gemm_fp8_2xAcc.py:10-50 (fp32 C; the gemm accumulates into a
    fragment that is added into a second one every 128 / block_K k-tiles)."""
    out_dtype = out_dtype or ("float" if two_acc else dtype)
    update_interval = 128 // block_K if block_K < 128 else 1

    @T.prim_func
    def main(A: T.Tensor((M, K), dtype), B: T.Tensor((N, K), dtype),
             C: T.Tensor((M, N), out_dtype)):
        with T.Kernel(T.ceildiv(N, block_N), T.ceildiv(M, block_M), threads=128) as (bx, by):
            A_shared = T.alloc_shared((block_M, block_K), dtype)
            B_shared = T.alloc_shared((block_N, block_K), dtype)
            C_local = T.alloc_fragment((block_M, block_N), "float")
            if two_acc:
                C_shared = T.alloc_shared((block_M, block_N), "float")
                C_acc = T.alloc_fragment((block_M, block_N), "float")
                T.clear(C_acc)
            T.clear(C_local)
            k_iters = T.ceildiv(K, block_K)
            for k in T.Pipelined(k_iters, num_stages=3):
                T.copy(A[by * block_M, k * block_K], A_shared)
                T.copy(B[bx * block_N, k * block_K], B_shared)
                T.gemm(A_shared, B_shared, C_local, transpose_B=True)
                if two_acc:
                    if (k + 1) % update_interval == 0:
                        for i, j in T.Parallel(block_M, block_N):
                            C_acc[i, j] += C_local[i, j]
                        T.clear(C_local)
            if two_acc:
                T.copy(C_acc, C_shared)
                T.copy(C_shared, C[by * block_M, bx * block_N])
            else:
                T.copy(C_local, C[by * block_M, bx * block_N])

    return main


def sigmoid(Block_w, Block_c, C, W, dtype="float32"):
    """tpu_demo/tpu_test_sigmoid_fp32.py:6-31."""
    shape = (C, W)

    @T.prim_func
    def main(G_in: T.Tensor(shape, dtype), G_out: T.Tensor(shape, dtype)):
        with T.Kernel(T.ceildiv(C, Block_c), T.ceildiv(W, Block_w), is_cpu=True) as (bx, by):
            tile = (Block_c, Block_w)
            x = T.alloc_shared(tile, dtype)
            out = T.alloc_shared(tile, dtype)
            work0 = T.alloc_shared(tile, dtype)
            work1 = T.alloc_shared(tile, dtype)
            coeff = T.alloc_shared([64, 32], dtype)
            table = T.alloc_shared([64, 192], dtype)
            T.ppl_copy(G_in[bx * Block_c, by * Block_w], x)
            T.ppl_sigmoid(out, x, work0, work1, coeff, table)
            T.ppl_copy(out, G_out[bx * Block_c, by * Block_w])

    return main


def gather(num_rows, hidden_size, num_indices, dtype="float32"):
    """tpu_demo/tpu_test_gather_fp32.py:8-18."""

    @T.prim_func
    def main(Param: T.Tensor((num_rows, hidden_size), dtype),
             Index: T.Tensor((num_indices, 1), "uint32"),
             Output: T.Tensor((num_indices, hidden_size), dtype)):
        with T.Kernel(1, 1, is_cpu=True) as (bx, by):
            T.ppl_gather(Output, Param, Index, num_rows)

    return main


def topk(length, K, descended=True, dtype="float32"):
    """tpu_demo/tpu_test_topk_fp32.py:6-18."""

    @T.prim_func
    def main(Input: T.Tensor((length,), dtype), Output: T.Tensor((length,), dtype),
             Indices: T.Tensor((length,), "int32")):
        with T.Kernel(1, 1, is_cpu=True) as (bx, by):
            T.ppl_topk(Output, Indices, Input, K, 1 if descended else 0, length)

    return main


def row_reduce(M, N, block_M, block_N, op="max", dtype="float16", accum_dtype="float16"):
    """tpu_demo/tpu_test_reduce_max.py and tpu_test_reduce_sum.py."""

    @T.prim_func
    def main(X: T.Tensor((M, N), dtype), Y: T.Tensor((M, 1), accum_dtype)):
        with T.Kernel(1, T.ceildiv(M, block_M), is_cpu=True) as (bx, by):
            X_shared = T.alloc_shared((block_M, block_N), dtype)
            Y_shared = T.alloc_shared((block_M, 1), accum_dtype)
            if op == "sum":
                T.ppl_fill(Y_shared, T.float32(0))
            T.ppl_copy(X[by * block_M, 0], X_shared)
            if op == "max":
                T.ppl_reduce_max(X_shared, Y_shared, 1, True)
            else:
                T.ppl_reduce_sum(X_shared, Y_shared, 1)
            T.ppl_copy(Y_shared, Y[by * block_M, 0])

    return main


def _rope_tile(x_src, cos_src, sin_src, dst, shape, dtype):
    x = T.alloc_shared(shape, dtype)
    c = T.alloc_shared(shape, dtype)
    s = T.alloc_shared(shape, dtype)
    T.ppl_copy(x_src, x)
    T.ppl_copy(cos_src, c)
    T.ppl_copy(sin_src, s)
    x_cos = T.alloc_shared(shape, dtype)
    x_sin = T.alloc_shared(shape, dtype)
    x_neg = T.alloc_shared(shape, dtype)
    x_neg_sin = T.alloc_shared(shape, dtype)
    T.ppl_mul(x_cos, x, c)
    T.ppl_mul(x_sin, x, s)
    T.ppl_mul_C(x_neg, x, T.float32(-1.0))
    T.ppl_mul(x_neg_sin, x_neg, s)
    out = T.alloc_shared(shape, dtype)
    T.ppl_rope_add(out, x_cos, x_neg_sin, x_cos, x_sin)
    T.ppl_copy(out, dst)


def rope(Block_c, Block_w, C, W, dtype="bfloat16", out_first=False):
    """tpu_test_rope_bf16.py:5-51 (G_in, G_cos, G_sin, G_out); out_first gives the parameter
    order of tpu_demo/ppl/rope/rope_{bf16,fp16,fp32}.py:8-13 (G_out, G_in, G_cos, G_sin)."""
    shape = (C, W)

    def body(G_in, G_cos, G_sin, G_out):
        with T.Kernel(T.ceildiv(C, Block_c), T.ceildiv(W, Block_w), is_cpu=True) as (bx, by):
            _rope_tile(G_in[bx * Block_c, by * Block_w], G_cos[bx * Block_c, by * Block_w],
                       G_sin[bx * Block_c, by * Block_w], G_out[bx * Block_c, by * Block_w],
                       (Block_c, Block_w), dtype)

    if out_first:

        @T.prim_func
        def rope_out_first(G_out: T.Tensor(shape, dtype), G_in: T.Tensor(shape, dtype),
                           G_cos: T.Tensor(shape, dtype), G_sin: T.Tensor(shape, dtype)):
            body(G_in, G_cos, G_sin, G_out)

        return rope_out_first

    @T.prim_func
    def rope_kernel(G_in: T.Tensor(shape, dtype), G_cos: T.Tensor(shape, dtype),
                    G_sin: T.Tensor(shape, dtype), G_out: T.Tensor(shape, dtype)):
        body(G_in, G_cos, G_sin, G_out)

    return rope_kernel


def rope_qk(tokens, heads_q, heads_k, W, Block_t=64, dtype="bfloat16"):
    """q [tokens, heads_q, W] and k [tokens, heads_k, W] rotated with one [tokens, W] table pair."""

    @T.prim_func
    def rope_qk_kernel(Q: T.Tensor((tokens, heads_q, W), dtype),
                       K: T.Tensor((tokens, heads_k, W), dtype),
                       COS: T.Tensor((tokens, W), dtype), SIN: T.Tensor((tokens, W), dtype),
                       Q_out: T.Tensor((tokens, heads_q, W), dtype),
                       K_out: T.Tensor((tokens, heads_k, W), dtype)):
        for X, Y, H in ((Q, Q_out, heads_q), (K, K_out, heads_k)):
            with T.Kernel(T.ceildiv(tokens, Block_t), H, is_cpu=True) as (bx, by):
                tok = slice(bx * Block_t, (bx + 1) * Block_t)
                _rope_tile(X[tok, by, :], COS[tok, :], SIN[tok, :], Y[tok, by, :], (Block_t, W),
                           dtype)

    return rope_qk_kernel


def swi_glu(Block_w, Block_c, C, W, dtype="bfloat16"):
    """tpu_test_swiglu_bf16.py:5-54; dtype float32 gives tpu_test_swiglu_fp32.py (tiles loaded
    and stored as fp32 directly)."""
    shape = (C, W)
    acc = "float32"
    f32 = dtype == "float32"

    @T.prim_func
    def swiglu(G_in: T.Tensor(shape, dtype), G_right: T.Tensor(shape, dtype),
               G_out: T.Tensor(shape, dtype)):
        with T.Kernel(T.ceildiv(C, Block_c), T.ceildiv(W, Block_w), is_cpu=True) as (bx, by):
            tile = (Block_c, Block_w)
            g16 = T.alloc_shared(tile, dtype)
            u16 = T.alloc_shared(tile, dtype)
            g = g16 if f32 else T.alloc_shared(tile, acc)
            u = u16 if f32 else T.alloc_shared(tile, acc)
            e = T.alloc_shared(tile, acc)
            ones = T.alloc_shared(tile, acc)
            den = T.alloc_shared(tile, acc)
            sig = T.alloc_shared(tile, acc)
            out = T.alloc_shared(tile, acc)
            o16 = out if f32 else T.alloc_shared(tile, dtype)
            T.ppl_fill(ones, T.float32(1.0))
            T.ppl_copy(G_in[bx * Block_c, by * Block_w], g16)
            T.ppl_copy(G_right[bx * Block_c, by * Block_w], u16)
            if not f32:
                T.ppl_copy(g16, g)
                T.ppl_copy(u16, u)
            T.ppl_mul_C(e, g, T.float32(-1.0))
            T.ppl_exp2(e)  # natural exp on BM1690 (customize.py:328-329)
            T.ppl_add(den, e, ones)
            T.ppl_div(sig, g, den)
            T.ppl_mul(out, u, sig)
            if not f32:
                T.ppl_copy(out, o16)
            T.ppl_copy(o16, G_out[bx * Block_c, by * Block_w])

    return swiglu


def deepseek_mlp(Block_bs, Block_h, Block_i, batch_seq, hidden_size, intermediate_size,
                 dtype="bfloat16"):
    """The program structure of tpu_demo/ppl/mlp/mlp_bf16.py:10-141 (DeepSeek-V3 MLP): per
    (row block, hidden block, intermediate block) the gate and up projections
    x_blk @ W_blk^T are ppl_gemm into 16-bit tiles, converted to fp32; SiLU(gate) = gate /
    (1 + exp(-gate)) times up in fp32, rounded to the 16-bit type; the down projection
    gated @ Wd_blk^T is stored to the output block. Parameters: output [batch_seq, hidden],
    x [batch_seq, hidden], gate_weight, up_weight [intermediate, hidden], down_weight
    [hidden, intermediate]."""
    acc = "float32"

    @T.macro
    def silu(g: T.Tensor((Block_bs, Block_i), acc), out: T.Tensor((Block_bs, Block_i), acc),
             neg: T.Tensor((Block_bs, Block_i), acc), ones: T.Tensor((Block_bs, Block_i), acc),
             den: T.Tensor((Block_bs, Block_i), acc)):
        T.ppl_mul_C(neg, g, T.float32(-1.0))
        T.ppl_exp2(neg)  # natural exp on BM1690 (customize.py:328-329)
        T.ppl_add(den, neg, ones)
        T.ppl_div(out, g, den)

    @T.prim_func
    def main(output: T.Tensor((batch_seq, hidden_size), dtype),
             x: T.Tensor((batch_seq, hidden_size), dtype),
             gate_weight: T.Tensor((intermediate_size, hidden_size), dtype),
             up_weight: T.Tensor((intermediate_size, hidden_size), dtype),
             down_weight: T.Tensor((hidden_size, intermediate_size), dtype)):
        with T.Kernel(T.ceildiv(batch_seq, Block_bs), T.ceildiv(hidden_size, Block_h),
                      T.ceildiv(intermediate_size, Block_i), is_cpu=True) as (bx, by, bz):
            xb = T.alloc_shared((Block_bs, Block_h), dtype)
            wg = T.alloc_shared((Block_i, Block_h), dtype)
            wu = T.alloc_shared((Block_i, Block_h), dtype)
            wd = T.alloc_shared((Block_h, Block_i), dtype)
            g16 = T.alloc_shared((Block_bs, Block_i), dtype)
            u16 = T.alloc_shared((Block_bs, Block_i), dtype)
            d16 = T.alloc_shared((Block_bs, Block_h), dtype)
            g32 = T.alloc_shared((Block_bs, Block_i), acc)
            u32 = T.alloc_shared((Block_bs, Block_i), acc)
            s32 = T.alloc_shared((Block_bs, Block_i), acc)
            h32 = T.alloc_shared((Block_bs, Block_i), acc)
            h16 = T.alloc_shared((Block_bs, Block_i), dtype)
            neg = T.alloc_shared((Block_bs, Block_i), acc)
            ones = T.alloc_shared((Block_bs, Block_i), acc)
            den = T.alloc_shared((Block_bs, Block_i), acc)
            T.ppl_fill(ones, T.float32(1.0))
            T.ppl_copy(x[bx * Block_bs:(bx + 1) * Block_bs, by * Block_h:(by + 1) * Block_h], xb)
            T.ppl_copy(gate_weight[bz * Block_i:(bz + 1) * Block_i,
                                   by * Block_h:(by + 1) * Block_h], wg)
            T.ppl_copy(up_weight[bz * Block_i:(bz + 1) * Block_i,
                                 by * Block_h:(by + 1) * Block_h], wu)
            T.ppl_copy(down_weight[by * Block_h:(by + 1) * Block_h,
                                   bz * Block_i:(bz + 1) * Block_i], wd)
            T.ppl_gemm(xb, wg, g16, transpose_B=True)
            T.ppl_copy(g16, g32)
            silu(g32, s32, neg, ones, den)
            T.ppl_gemm(xb, wu, u16, transpose_B=True)
            T.ppl_copy(u16, u32)
            T.ppl_mul(h32, s32, u32)
            T.ppl_copy(h32, h16)
            T.ppl_gemm(h16, wd, d16, transpose_B=True)
            T.ppl_copy(d16, output[bx * Block_bs:(bx + 1) * Block_bs,
                                   by * Block_h:(by + 1) * Block_h])

    return main


def deepseek_mlp_fp32(Block_bs, Block_h, Block_i, batch_seq, hidden_size, intermediate_size,
                      gemm_dtype="bfloat16"):
    """The program structure of tpu_demo/ppl/mlp/mlp_fp32.py:7-120: fp32 parameters and tiles;
    the x / weight tiles are copied to bf16 tiles for the three ppl_gemm (transpose_B, bf16
    results, :95-114), gate and up read back as fp32, SiLU(gate) * up in fp32 rounded to bf16
    for the down projection, whose bf16 result is copied to the fp32 output block (:116-120)."""
    acc = "float32"
    gdt = gemm_dtype

    @T.macro
    def silu(g: T.Tensor((Block_bs, Block_i), acc), out: T.Tensor((Block_bs, Block_i), acc),
             neg: T.Tensor((Block_bs, Block_i), acc), ones: T.Tensor((Block_bs, Block_i), acc),
             den: T.Tensor((Block_bs, Block_i), acc)):
        T.ppl_mul_C(neg, g, T.float32(-1.0))
        T.ppl_exp2(neg)  # natural exp on BM1690 (customize.py:328-329)
        T.ppl_add(den, neg, ones)
        T.ppl_div(out, g, den)

    @T.prim_func
    def main(output: T.Tensor((batch_seq, hidden_size), acc),
             x: T.Tensor((batch_seq, hidden_size), acc),
             gate_weight: T.Tensor((intermediate_size, hidden_size), acc),
             up_weight: T.Tensor((intermediate_size, hidden_size), acc),
             down_weight: T.Tensor((hidden_size, intermediate_size), acc)):
        with T.Kernel(T.ceildiv(batch_seq, Block_bs), T.ceildiv(hidden_size, Block_h),
                      T.ceildiv(intermediate_size, Block_i), is_cpu=True) as (bx, by, bz):
            x32 = T.alloc_shared((Block_bs, Block_h), acc)
            wg32 = T.alloc_shared((Block_i, Block_h), acc)
            wu32 = T.alloc_shared((Block_i, Block_h), acc)
            wd32 = T.alloc_shared((Block_h, Block_i), acc)
            g32 = T.alloc_shared((Block_bs, Block_i), acc)
            u32 = T.alloc_shared((Block_bs, Block_i), acc)
            d32 = T.alloc_shared((Block_bs, Block_h), acc)
            s32 = T.alloc_shared((Block_bs, Block_i), acc)
            h32 = T.alloc_shared((Block_bs, Block_i), acc)
            neg = T.alloc_shared((Block_bs, Block_i), acc)
            ones = T.alloc_shared((Block_bs, Block_i), acc)
            den = T.alloc_shared((Block_bs, Block_i), acc)
            T.ppl_fill(ones, T.float32(1.0))
            T.ppl_copy(x[bx * Block_bs:(bx + 1) * Block_bs, by * Block_h:(by + 1) * Block_h], x32)
            T.ppl_copy(gate_weight[bz * Block_i:(bz + 1) * Block_i,
                                   by * Block_h:(by + 1) * Block_h], wg32)
            T.ppl_copy(up_weight[bz * Block_i:(bz + 1) * Block_i,
                                 by * Block_h:(by + 1) * Block_h], wu32)
            T.ppl_copy(down_weight[by * Block_h:(by + 1) * Block_h,
                                   bz * Block_i:(bz + 1) * Block_i], wd32)
            xb = T.alloc_shared((Block_bs, Block_h), gdt)
            wg = T.alloc_shared((Block_i, Block_h), gdt)
            wu = T.alloc_shared((Block_i, Block_h), gdt)
            wd = T.alloc_shared((Block_h, Block_i), gdt)
            g16 = T.alloc_shared((Block_bs, Block_i), gdt)
            u16 = T.alloc_shared((Block_bs, Block_i), gdt)
            h16 = T.alloc_shared((Block_bs, Block_i), gdt)
            d16 = T.alloc_shared((Block_bs, Block_h), gdt)
            T.ppl_copy(x32, xb)
            T.ppl_copy(wg32, wg)
            T.ppl_copy(wu32, wu)
            T.ppl_copy(wd32, wd)
            T.ppl_gemm(xb, wg, g16, transpose_B=True)
            T.ppl_copy(g16, g32)
            silu(g32, s32, neg, ones, den)
            T.ppl_gemm(xb, wu, u16, transpose_B=True)
            T.ppl_copy(u16, u32)
            T.ppl_mul(h32, s32, u32)
            T.ppl_copy(h32, h16)
            T.ppl_gemm(h16, wd, d16, transpose_B=True)
            T.ppl_copy(d16, d32)
            T.ppl_copy(d32, output[bx * Block_bs:(bx + 1) * Block_bs,
                                   by * Block_h:(by + 1) * Block_h])

    return main


def flashattn(batch, heads, seq_len, dim, is_causal, block_M=128, block_N=128,
              dtype="bfloat16", gemm_dtype=None, kv_blocks=None):
    """tpu_test_flashattn_bf16.py:14-135 (fp16 twin); dtype float32 with gemm_dtype float16
    gives tpu_test_flashattn_fp32.py: Q, K, V tiles and P copied to fp16 tiles for the two
    ppl_gemm, softmax state, acc_o and the output in fp32. kv_blocks (non-causal) sets the
    number of key blocks the loop visits (default all: a program over fewer attends to a
    prefix of the keys, which the recogniser rejects)."""
    scale = (1.0 / dim) ** 0.5
    shape = [batch, seq_len, heads, dim]
    acc = "float32"
    gdt = gemm_dtype or dtype

    @T.prim_func
    def fa(Q: T.Tensor(shape, dtype), K: T.Tensor(shape, dtype), V: T.Tensor(shape, dtype),
           Output: T.Tensor(shape, dtype)):
        with T.Kernel(T.ceildiv(seq_len, block_M), heads, batch, is_cpu=True) as (bx, by, bz):
            q_s = T.alloc_shared([block_M, dim], dtype)
            k_s = T.alloc_shared([block_N, dim], dtype)
            v_s = T.alloc_shared([block_N, dim], dtype)
            q_g = q_s if gdt == dtype else T.alloc_shared([block_M, dim], gdt)
            k_g = k_s if gdt == dtype else T.alloc_shared([block_N, dim], gdt)
            v_g = v_s if gdt == dtype else T.alloc_shared([block_N, dim], gdt)
            o_s = T.alloc_shared([block_M, dim], dtype)
            s = T.alloc_shared([block_M, block_N], acc)
            p = T.alloc_shared([block_M, block_N], gdt)
            o = T.alloc_shared([block_M, dim], acc)
            m = T.alloc_shared([block_M, 1], acc)
            m_prev = T.alloc_shared([block_M, 1], acc)
            alpha = T.alloc_shared([block_M, 1], acc)
            rsum = T.alloc_shared([block_M, 1], acc)
            l = T.alloc_shared([block_M, 1], acc)
            T.ppl_copy(Q[bz, bx * block_M:(bx + 1) * block_M, by, :], q_s)
            T.ppl_fill(o, T.float32(0))
            T.ppl_fill(l, T.float32(0))
            T.ppl_fill(m, -T.infinity(acc))
            n_kv = (T.min(T.ceildiv(seq_len, block_N), T.ceildiv((bx + 1) * block_M, block_N))
                    if is_causal else kv_blocks or T.ceildiv(seq_len, block_N))
            for k in T.Pipelined(n_kv, num_stages=2):
                T.ppl_copy(K[bz, k * block_N:(k + 1) * block_N, by, :], k_s)
                T.ppl_fill(s, T.float32(0))
                if gdt != dtype:
                    T.ppl_copy(q_s, q_g)
                    T.ppl_copy(k_s, k_g)
                T.ppl_gemm(q_g, k_g, s, transpose_B=True)
                T.ppl_copy(m, m_prev)
                T.ppl_fill(m, -T.infinity(acc))
                T.ppl_reduce_max(s, m, dim=1, clear=False)
                T.ppl_subtract(alpha, m_prev, m)
                T.ppl_mul_C(alpha, alpha, scale)
                T.ppl_exp2(alpha)
                T.ppl_subtract(s, s, m)
                T.ppl_mul_C(s, s, scale)
                T.ppl_exp2(s)
                T.ppl_reduce_sum(s, rsum, dim=1)
                T.ppl_mul(l, l, alpha)
                T.ppl_add(l, l, rsum)
                T.ppl_copy(s, p)
                T.ppl_mul(o, o, alpha)
                T.ppl_copy(V[bz, k * block_N:(k + 1) * block_N, by, :], v_s)
                if gdt != dtype:
                    T.ppl_copy(v_s, v_g)
                T.ppl_gemm(p, v_g, o)
            T.ppl_div(o, o, l)
            T.ppl_copy(o, o_s)
            T.ppl_copy(o_s, Output[bz, bx * block_M:(bx + 1) * block_M, by, :])

    return fa


def flashattn_gqa(batch, heads, seq_len, dim, is_causal, groups=1, block_M=128, block_N=128,
                  dtype="float16"):
    """The upstream program structure of examples/flash_attention/example_gqa_fwd_bshd.py:62-178
    (groups=1: example_mha_fwd_bshd.py): T.copy / T.gemm tiles, the causal mask written into the
    scores with if_then_else before Q K^T accumulates onto them, softmax in the exp2 domain with
    the scale folded in (scale * log2 e), query head by reading K/V head by // groups."""
    scale = (1.0 / dim) ** 0.5 * 1.44269504
    head_kv = heads // groups
    q_shape = [batch, seq_len, heads, dim]
    kv_shape = [batch, seq_len, head_kv, dim]
    acc = "float"

    @T.prim_func
    def main(Q: T.Tensor(q_shape, dtype), K: T.Tensor(kv_shape, dtype),
             V: T.Tensor(kv_shape, dtype), Output: T.Tensor(q_shape, dtype)):
        with T.Kernel(T.ceildiv(seq_len, block_M), heads, batch, threads=128) as (bx, by, bz):
            q_s = T.alloc_shared([block_M, dim], dtype)
            k_s = T.alloc_shared([block_N, dim], dtype)
            v_s = T.alloc_shared([block_N, dim], dtype)
            o_s = T.alloc_shared([block_M, dim], dtype)
            s = T.alloc_fragment([block_M, block_N], acc)
            s_cast = T.alloc_fragment([block_M, block_N], dtype)
            o = T.alloc_fragment([block_M, dim], acc)
            m = T.alloc_fragment([block_M], acc)
            m_prev = T.alloc_fragment([block_M], acc)
            alpha = T.alloc_fragment([block_M], acc)
            rsum = T.alloc_fragment([block_M], acc)
            l = T.alloc_fragment([block_M], acc)
            T.copy(Q[bz, bx * block_M:(bx + 1) * block_M, by, :], q_s)
            T.fill(o, 0)
            T.fill(l, 0)
            T.fill(m, -T.infinity(acc))
            n_kv = (T.min(T.ceildiv(seq_len, block_N), T.ceildiv((bx + 1) * block_M, block_N))
                    if is_causal else T.ceildiv(seq_len, block_N))
            for k in T.Pipelined(n_kv, num_stages=2):
                T.copy(K[bz, k * block_N:(k + 1) * block_N, by // groups, :], k_s)
                if is_causal:
                    for i, j in T.Parallel(block_M, block_N):
                        s[i, j] = T.if_then_else(bx * block_M + i >= k * block_N + j, 0,
                                                 -T.infinity(acc))
                else:
                    T.clear(s)
                T.gemm(q_s, k_s, s, transpose_B=True, policy=T.GemmWarpPolicy.FullRow)
                T.copy(m, m_prev)
                T.fill(m, -T.infinity(acc))
                T.reduce_max(s, m, dim=1, clear=False)
                for i in T.Parallel(block_M):
                    alpha[i] = T.exp2(m_prev[i] * scale - m[i] * scale)
                for i, j in T.Parallel(block_M, block_N):
                    s[i, j] = T.exp2(s[i, j] * scale - m[i] * scale)
                T.reduce_sum(s, rsum, dim=1)
                for i in T.Parallel(block_M):
                    l[i] = l[i] * alpha[i] + rsum[i]
                T.copy(s, s_cast)
                for i, j in T.Parallel(block_M, dim):
                    o[i, j] *= alpha[i]
                T.copy(V[bz, k * block_N:(k + 1) * block_N, by // groups, :], v_s)
                T.gemm(s_cast, v_s, o, policy=T.GemmWarpPolicy.FullRow)
            for i, j in T.Parallel(block_M, dim):
                o[i, j] /= l[i]
            T.copy(o, o_s)
            T.copy(o_s, Output[bz, bx * block_M:(bx + 1) * block_M, by, :])

    return main


def flashattn_bhsd(batch, heads, seq_q, seq_kv, dim, is_causal, block_M=128, block_N=128,
                   dtype="float16"):
    """The program structure of examples/flash_attention/example_mha_fwd_bhsd.py:30-158:
    head-major Q, Output [batch, heads, seq_q, dim] and K, V [batch, heads, seq_kv, dim]; the
    score, softmax, rescale and P V steps written as @T.macro helpers with tile-buffer
    annotations; the causal mask offset by past_len = seq_kv - seq_q."""
    scale = (1.0 / dim) ** 0.5 * 1.44269504
    q_shape = [batch, heads, seq_q, dim]
    kv_shape = [batch, heads, seq_kv, dim]
    acc = "float"

    @T.macro
    def scores(K: T.Tensor(kv_shape, dtype), q_s: T.SharedBuffer([block_M, dim], dtype),
               k_s: T.SharedBuffer([block_N, dim], dtype),
               s: T.FragmentBuffer([block_M, block_N], acc), k: T.int32, bx: T.int32,
               by: T.int32, bz: T.int32):
        past_len = seq_kv - seq_q
        T.copy(K[bz, by, k * block_N:(k + 1) * block_N, :], k_s)
        if is_causal:
            for i, j in T.Parallel(block_M, block_N):
                s[i, j] = T.if_then_else(bx * block_M + i + past_len >= k * block_N + j, 0,
                                         -T.infinity(acc))
        else:
            T.clear(s)
        T.gemm(q_s, k_s, s, transpose_B=True, policy=T.GemmWarpPolicy.FullRow)

    @T.macro
    def online_softmax(s: T.FragmentBuffer([block_M, block_N], acc),
                       s_cast: T.FragmentBuffer([block_M, block_N], dtype),
                       m: T.FragmentBuffer([block_M], acc), m_prev: T.FragmentBuffer([block_M], acc),
                       alpha: T.FragmentBuffer([block_M], acc),
                       rsum: T.FragmentBuffer([block_M], acc), l: T.FragmentBuffer([block_M], acc)):
        T.copy(m, m_prev)
        T.fill(m, -T.infinity(acc))
        T.reduce_max(s, m, dim=1, clear=False)
        for i in T.Parallel(block_M):
            alpha[i] = T.exp2(m_prev[i] * scale - m[i] * scale)
        for i, j in T.Parallel(block_M, block_N):
            s[i, j] = T.exp2(s[i, j] * scale - m[i] * scale)
        T.reduce_sum(s, rsum, dim=1)
        for i in T.Parallel(block_M):
            l[i] = l[i] * alpha[i] + rsum[i]
        T.copy(s, s_cast)

    @T.macro
    def rescale(o: T.FragmentBuffer([block_M, dim], acc), alpha: T.FragmentBuffer([block_M], acc)):
        for i, j in T.Parallel(block_M, dim):
            o[i, j] *= alpha[i]

    @T.macro
    def pv(V: T.Tensor(kv_shape, dtype), v_s: T.SharedBuffer([block_N, dim], dtype),
           s_cast: T.FragmentBuffer([block_M, block_N], dtype),
           o: T.FragmentBuffer([block_M, dim], acc), k: T.int32, by: T.int32, bz: T.int32):
        T.copy(V[bz, by, k * block_N:(k + 1) * block_N, :], v_s)
        T.gemm(s_cast, v_s, o, policy=T.GemmWarpPolicy.FullRow)

    @T.prim_func
    def main(Q: T.Tensor(q_shape, dtype), K: T.Tensor(kv_shape, dtype),
             V: T.Tensor(kv_shape, dtype), Output: T.Tensor(q_shape, dtype)):
        with T.Kernel(T.ceildiv(seq_q, block_M), heads, batch, threads=128) as (bx, by, bz):
            q_s = T.alloc_shared([block_M, dim], dtype)
            k_s = T.alloc_shared([block_N, dim], dtype)
            v_s = T.alloc_shared([block_N, dim], dtype)
            o_s = T.alloc_shared([block_M, dim], dtype)
            s = T.alloc_fragment([block_M, block_N], acc)
            s_cast = T.alloc_fragment([block_M, block_N], dtype)
            o = T.alloc_fragment([block_M, dim], acc)
            m = T.alloc_fragment([block_M], acc)
            m_prev = T.alloc_fragment([block_M], acc)
            alpha = T.alloc_fragment([block_M], acc)
            rsum = T.alloc_fragment([block_M], acc)
            l = T.alloc_fragment([block_M], acc)
            T.copy(Q[bz, by, bx * block_M:(bx + 1) * block_M, :], q_s)
            T.fill(o, 0)
            T.fill(l, 0)
            T.fill(m, -T.infinity(acc))
            n_kv = (T.min(T.ceildiv(seq_kv, block_N), T.ceildiv((bx + 1) * block_M, block_N))
                    if is_causal else T.ceildiv(seq_kv, block_N))
            for k in T.Pipelined(n_kv, num_stages=2):
                scores(K, q_s, k_s, s, k, bx, by, bz)
                online_softmax(s, s_cast, m, m_prev, alpha, rsum, l)
                rescale(o, alpha)
                pv(V, v_s, s_cast, o, k, by, bz)
            for i, j in T.Parallel(block_M, dim):
                o[i, j] /= l[i]
            T.copy(o, o_s)
            T.copy(o_s, Output[bz, by, bx * block_M:(bx + 1) * block_M, :])

    return main


def mha_inference(batch, heads, seqlen_q, seqlen_kv, dim, is_causal=False, block_M=128,
                  block_N=64, num_split=4, dtype="float16"):
    """The program structure of examples/flash_attention/example_mha_inference.py:11-203:
    split-KV attention for short query blocks over long key ranges. Kernel 1 (flash_attn_split,
    grid [ceil(seqlen_q / block_M), heads * batch, num_split]) runs the online softmax of one
    query block over the split's seqlen_kv // num_split keys and stores the normalised partial
    output in Output_partial [batch, seqlen_q, heads, num_split, dim] and its log2 sum-exp in
    glse [batch, heads, num_split, seqlen_q]; kernel 2 (combine) merges the splits into Output.
    Q, Output [batch, seqlen_q, heads, dim]; K, V [batch, seqlen_kv, heads, dim]; Output is
    parameter 5."""
    scale = (1.0 / dim) ** 0.5 * 1.44269504
    shape_q = [batch, seqlen_q, heads, dim]
    shape_kv = [batch, seqlen_kv, heads, dim]
    part_shape = [batch, seqlen_q, heads, num_split, dim]
    acc = "float"
    per = seqlen_kv // num_split

    @T.macro
    def scores(K: T.Tensor(shape_kv, dtype), q_s: T.SharedBuffer([block_M, dim], dtype),
               k_s: T.SharedBuffer([block_N, dim], dtype),
               s: T.FragmentBuffer([block_M, block_N], acc), k: T.int32, mid: T.int32,
               hid: T.int32, bid: T.int32, sid: T.int32):
        T.copy(K[bid, per * sid + k * block_N:per * sid + (k + 1) * block_N, hid, :], k_s)
        if is_causal:
            for i, j in T.Parallel(block_M, block_N):
                s[i, j] = T.if_then_else(mid * block_M + i >= k * block_N + j, 0,
                                         -T.infinity(acc))
        else:
            T.clear(s)
        T.gemm(q_s, k_s, s, transpose_B=True, policy=T.GemmWarpPolicy.FullRow)

    @T.macro
    def pv(V: T.Tensor(shape_kv, dtype), v_s: T.SharedBuffer([block_M, dim], dtype),
           s_cast: T.FragmentBuffer([block_M, block_N], dtype),
           o: T.FragmentBuffer([block_M, dim], acc), k: T.int32, hid: T.int32, bid: T.int32,
           sid: T.int32):
        T.copy(V[bid, per * sid + k * block_N:per * sid + (k + 1) * block_N, hid, :], v_s)
        T.gemm(s_cast, v_s, o, policy=T.GemmWarpPolicy.FullRow)

    @T.macro
    def softmax(s: T.FragmentBuffer([block_M, block_N], acc),
                s_cast: T.FragmentBuffer([block_M, block_N], dtype),
                m: T.FragmentBuffer([block_M], acc), m_prev: T.FragmentBuffer([block_M], acc),
                alpha: T.FragmentBuffer([block_M], acc), rsum: T.FragmentBuffer([block_M], acc),
                l: T.FragmentBuffer([block_M], acc)):
        T.copy(m, m_prev)
        T.fill(m, -T.infinity(acc))
        T.reduce_max(s, m, dim=1, clear=False)
        for i in T.Parallel(block_M):
            alpha[i] = T.exp2(m_prev[i] * scale - m[i] * scale)
        for i, j in T.Parallel(block_M, block_N):
            s[i, j] = T.exp2(s[i, j] * scale - m[i] * scale)
        T.reduce_sum(s, rsum, dim=1)
        for i in T.Parallel(block_M):
            l[i] = l[i] * alpha[i] + rsum[i]
        T.copy(s, s_cast)

    @T.macro
    def rescale(o: T.FragmentBuffer([block_M, dim], acc), alpha: T.FragmentBuffer([block_M], acc)):
        for i, j in T.Parallel(block_M, dim):
            o[i, j] *= alpha[i]

    @T.macro
    def flash_attn_split(Q: T.Tensor(shape_q, dtype), K: T.Tensor(shape_kv, dtype),
                         V: T.Tensor(shape_kv, dtype),
                         glse: T.Tensor([batch, heads, num_split, seqlen_q], dtype),
                         Output_partial: T.Tensor(part_shape, dtype)):
        with T.Kernel(T.ceildiv(seqlen_q, block_M), heads * batch, num_split,
                      threads=128) as (bx, by, bz):
            q_s = T.alloc_shared([block_M, dim], dtype)
            k_s = T.alloc_shared([block_N, dim], dtype)
            v_s = T.alloc_shared([block_N, dim], dtype)
            o_s = T.alloc_shared([block_M, dim], dtype)
            s = T.alloc_fragment([block_M, block_N], acc)
            s_cast = T.alloc_fragment([block_M, block_N], dtype)
            o = T.alloc_fragment([block_M, dim], acc)
            m = T.alloc_fragment([block_M], acc)
            m_prev = T.alloc_fragment([block_M], acc)
            alpha = T.alloc_fragment([block_M], acc)
            rsum = T.alloc_fragment([block_M], acc)
            l = T.alloc_fragment([block_M], acc)
            mid = bx
            hid = by % heads
            bid = by // heads
            sid = bz
            T.copy(Q[bid, mid * block_M:(mid + 1) * block_M, hid, :], q_s)
            T.fill(o, 0)
            T.fill(l, 0)
            T.fill(m, -T.infinity(acc))
            n_kv = (T.min(T.ceildiv(seqlen_kv, block_N), T.ceildiv((mid + 1) * block_M, block_N))
                    if is_causal else T.ceildiv(per, block_N))
            for k in T.Pipelined(n_kv, num_stages=2):
                scores(K, q_s, k_s, s, k, mid, hid, bid, sid)
                softmax(s, s_cast, m, m_prev, alpha, rsum, l)
                rescale(o, alpha)
                pv(V, v_s, s_cast, o, k, hid, bid, sid)
            for i, j in T.Parallel(block_M, dim):
                o[i, j] /= l[i]
            for i in T.Parallel(block_M):
                l[i] = T.log2(l[i]) + m[i] * scale
            T.copy(l, glse[bid, hid, sid, mid * block_M:(mid + 1) * block_M])
            T.copy(o, o_s)
            T.copy(o_s, Output_partial[bid, mid * block_M:(mid + 1) * block_M, hid, sid, :])

    @T.macro
    def combine(glse: T.Tensor([batch, heads, num_split, seqlen_q], dtype),
                Output_partial: T.Tensor(part_shape, dtype), Output: T.Tensor(shape_q, dtype)):
        with T.Kernel(T.ceildiv(seqlen_q, block_M), heads, batch, threads=128) as (bx, by, bz):
            po = T.alloc_fragment([block_M, dim], dtype)
            po_s = T.alloc_shared([block_M, dim], dtype)
            o_acc = T.alloc_fragment([block_M, dim], acc)
            o_s = T.alloc_shared([block_M, dim], dtype)
            lse = T.alloc_fragment([num_split, block_M], dtype)
            lse_k = T.alloc_fragment([block_M], acc)
            lse_sum = T.alloc_fragment([block_M], acc)
            lse_max = T.alloc_fragment([block_M], acc)
            w = T.alloc_fragment([block_M], acc)
            T.clear(lse_sum)
            T.clear(o_acc)
            T.copy(glse[bz, by, :, bx * block_M:(bx + 1) * block_M], lse)
            T.reduce_max(lse, lse_max, dim=0, clear=False)
            for k in T.Pipelined(num_split):
                T.copy(lse[k, :], lse_k)
                for i in T.Parallel(block_M):
                    lse_sum[i] += T.exp2(lse_k[i] - lse_max[i])
            for i in T.Parallel(block_M):
                lse_sum[i] = T.log2(lse_sum[i]) + lse_max[i]
            for k in T.Pipelined(num_split, num_stages=2):
                T.copy(Output_partial[bz, bx * block_M:(bx + 1) * block_M, by, k, :], po_s)
                T.copy(po_s, po)
                T.copy(lse[k, :], lse_k)
                for i in T.Parallel(block_M):
                    w[i] = T.exp2(lse_k[i] - lse_sum[i])
                for i, j in T.Parallel(block_M, dim):
                    o_acc[i, j] += po[i, j] * w[i]
            T.copy(o_acc, o_s)
            T.copy(o_s, Output[bz, bx * block_M:(bx + 1) * block_M, by, :])

    @T.prim_func
    def main(Q: T.Tensor(shape_q, dtype), K: T.Tensor(shape_kv, dtype),
             V: T.Tensor(shape_kv, dtype),
             glse: T.Tensor([batch, heads, num_split, seqlen_q], dtype),
             Output_partial: T.Tensor(part_shape, dtype), Output: T.Tensor(shape_q, dtype)):
        flash_attn_split(Q, K, V, glse, Output_partial)
        combine(glse, Output_partial, Output)

    return main


def flashattn_varlen(batch, UQ, UKV, heads, dim, is_causal=False, groups=1, block_M=64,
                     block_N=64, dtype="float16"):
    """The program structure of examples/flash_attention/example_mha_fwd_varlen.py:222-358:
    unpadded Q [UQ, heads, dim], K/V [UKV, heads // groups, dim], int32 cu_seqlens of both
    sides, the scalar max_seqlen_q sizing the grid; tiles filled element by element with zeros
    past the sequence's end, scores pre-filled with -inf at out-of-range positions. is_causal
    reproduces the example's causal expression (:298-302), which masks a position only when
    it is both on or below the diagonal and out of range."""
    scale = (1.0 / dim) ** 0.5 * 1.44269504
    q_shape = [UQ, heads, dim]
    kv_shape = [UKV, heads // groups, dim]
    acc = "float"

    @T.prim_func
    def main(Q_unpad: T.Tensor(q_shape, dtype), K_unpad: T.Tensor(kv_shape, dtype),
             V_unpad: T.Tensor(kv_shape, dtype), cu_seqlens_q: T.Tensor([batch + 1], "int32"),
             cu_seqlens_k: T.Tensor([batch + 1], "int32"), max_seqlen_q: T.int32,
             Output_unpad: T.Tensor(q_shape, dtype)):
        with T.Kernel(T.ceildiv(max_seqlen_q, block_M), heads, batch, threads=32) as (bx, by, bz):
            q_s = T.alloc_shared([block_M, dim], dtype, "shared")
            k_s = T.alloc_shared([block_N, dim], dtype, "shared")
            v_s = T.alloc_shared([block_N, dim], dtype, "shared")
            o_s = T.alloc_shared([block_M, dim], dtype, "shared")
            s = T.alloc_fragment([block_M, block_N], acc)
            s_cast = T.alloc_fragment([block_M, block_N], dtype)
            o = T.alloc_fragment([block_M, dim], acc)
            m = T.alloc_fragment([block_M], acc)
            m_prev = T.alloc_fragment([block_M], acc)
            alpha = T.alloc_fragment([block_M], acc)
            rsum = T.alloc_fragment([block_M], acc)
            l = T.alloc_fragment([block_M], acc)
            hk = by // groups
            q_start, k_start = cu_seqlens_q[bz], cu_seqlens_k[bz]
            q_len = cu_seqlens_q[bz + 1] - q_start
            k_len = cu_seqlens_k[bz + 1] - k_start
            for i, d in T.Parallel(block_M, dim):
                if bx * block_M + i < q_len:
                    q_s[i, d] = Q_unpad[q_start + bx * block_M + i, by, d]
                else:
                    q_s[i, d] = 0
            T.fill(o, 0)
            T.fill(l, 0)
            T.fill(m, -T.infinity(acc))
            for k in T.Pipelined(T.ceildiv(k_len, block_N), num_stages=0):
                for i, d in T.Parallel(block_N, dim):
                    if k * block_N + i < k_len:
                        k_s[i, d] = K_unpad[k_start + k * block_N + i, hk, d]
                    else:
                        k_s[i, d] = 0
                if is_causal:
                    for i, j in T.Parallel(block_M, block_N):
                        s[i, j] = T.if_then_else(
                            (bx * block_M + i >= k * block_N + j) and
                            (bx * block_M + i >= q_len or k * block_N + j >= k_len),
                            -T.infinity(acc), 0)
                else:
                    for i, j in T.Parallel(block_M, block_N):
                        s[i, j] = T.if_then_else(
                            (bx * block_M + i >= q_len or k * block_N + j >= k_len),
                            -T.infinity(acc), 0)
                T.gemm(q_s, k_s, s, transpose_B=True, policy=T.GemmWarpPolicy.FullRow)
                T.copy(m, m_prev)
                T.fill(m, -T.infinity(acc))
                T.reduce_max(s, m, dim=1, clear=False)
                for i in T.Parallel(block_M):
                    alpha[i] = T.exp2(m_prev[i] * scale - m[i] * scale)
                for i, j in T.Parallel(block_M, block_N):
                    s[i, j] = T.exp2(s[i, j] * scale - m[i] * scale)
                T.reduce_sum(s, rsum, dim=1)
                for i in T.Parallel(block_M):
                    l[i] = l[i] * alpha[i] + rsum[i]
                T.copy(s, s_cast)
                for i, j in T.Parallel(block_M, dim):
                    o[i, j] *= alpha[i]
                for i, d in T.grid(block_N, dim):
                    if k * block_N + i < k_len:
                        v_s[i, d] = V_unpad[k_start + k * block_N + i, hk, d]
                    else:
                        v_s[i, d] = 0
                T.gemm(s_cast, v_s, o, policy=T.GemmWarpPolicy.FullRow)
            for i, j in T.Parallel(block_M, dim):
                o[i, j] /= l[i]
            T.copy(o, o_s)
            for i, d in T.Parallel(block_M, dim):
                if bx * block_M + i < q_len:
                    Output_unpad[q_start + bx * block_M + i, by, d] = o_s[i, d]

    return main


def mla_decode(batch, h_q, h_kv, max_seqlen_pad, dv, dpe, block_N, block_H, num_split,
               block_size, dtype="float16", kv_dtype=None, out_dtype=None):
    """Paged MLA decode with split-KV + LSE combine. ``kv_dtype="float8_e4m3"`` adds a trailing
    ``KV_scale: float32[1]`` parameter (values = fp8 * scale)."""
    kv_dtype = kv_dtype or dtype
    out_dtype = out_dtype or dtype
    fp8 = kv_dtype == "float8_e4m3"
    scale = (1.0 / (dv + dpe)) ** 0.5 * 1.44269504
    acc = "float32"
    assert h_kv == 1
    VB = min(block_H, h_q // h_kv)
    pages = max_seqlen_pad // block_size

    def split_kernel(Q, Q_pe, KV, K_pe, BT, SL, glse, Opart, KVS):
        with T.Kernel(batch, h_q // VB, num_split, threads=256) as (bx, by, bz):
            q_s = T.alloc_shared([block_H, dv], dtype)
            qpe_s = T.alloc_shared([block_H, dpe], dtype)
            kv_s = T.alloc_shared([block_N, dv], kv_dtype)
            kpe_s = T.alloc_shared([block_N, dpe], kv_dtype)
            s = T.alloc_fragment([block_H, block_N], acc)
            p = T.alloc_fragment([block_H, block_N], dtype)
            o = T.alloc_fragment([block_H, dv], acc)
            m = T.alloc_fragment([block_H], acc)
            m_prev = T.alloc_fragment([block_H], acc)
            alpha = T.alloc_fragment([block_H], acc)
            rsum = T.alloc_fragment([block_H], acc)
            l = T.alloc_fragment([block_H], acc)
            T.copy(Q[bx, by * VB:(by + 1) * VB, :], q_s)
            T.copy(Q_pe[bx, by * VB:(by + 1) * VB, :], qpe_s)
            T.fill(o, 0)
            T.fill(l, 0)
            T.fill(m, -T.infinity(acc))
            nblk = T.ceildiv(SL[bx], block_N)
            per = T.floordiv(nblk, num_split)
            rem = T.floormod(nblk, num_split)
            n_iter = per + T.if_then_else(bz < rem, 1, 0)
            start = (per * bz + T.min(bz, rem)) * block_N
            for k in T.Pipelined(n_iter, num_stages=2):
                tok = start + k * block_N
                row = BT[bx, tok // block_size] * block_size + tok % block_size
                T.copy(KV[row:row + block_N, 0, :], kv_s)
                T.copy(K_pe[row:row + block_N, 0, :], kpe_s)
                T.clear(s)
                T.gemm(q_s, kv_s, s, transpose_B=True)
                T.gemm(qpe_s, kpe_s, s, transpose_B=True)
                if fp8:
                    for i, j in T.Parallel(block_H, block_N):
                        s[i, j] = s[i, j] * KVS[0]
                T.copy(m, m_prev)
                T.fill(m, -T.infinity(acc))
                for i, j in T.Parallel(block_H, block_N):
                    s[i, j] = T.if_then_else(tok + j >= SL[bx], -T.infinity(acc), s[i, j])
                T.reduce_max(s, m, dim=1, clear=False)
                for i in T.Parallel(block_H):
                    alpha[i] = T.exp2(m_prev[i] * scale - m[i] * scale)
                for i, j in T.Parallel(block_H, block_N):
                    s[i, j] = T.exp2(s[i, j] * scale - m[i] * scale)
                T.reduce_sum(s, rsum, dim=1)
                T.copy(s, p)
                for i in T.Parallel(block_H):
                    l[i] = l[i] * alpha[i] + rsum[i]
                for i, j in T.Parallel(block_H, dv):
                    o[i, j] *= alpha[i]
                T.gemm(p, kv_s, o)
            for i, j in T.Parallel(block_H, dv):
                o[i, j] /= l[i]
                if fp8:
                    o[i, j] = o[i, j] * KVS[0]
            for i in T.Parallel(block_H):
                l[i] = T.log2(l[i]) + m[i] * scale
            T.copy(l, glse[bx, by * VB:(by + 1) * VB, bz])
            T.copy(o, Opart[bx, by * VB:(by + 1) * VB, bz, :])

    def combine(glse, Opart, Output):
        with T.Kernel(h_q, batch, threads=128) as (by, bz):
            acc_o = T.alloc_fragment([dv], acc)
            part = T.alloc_fragment([dv], acc)
            lse_max = T.alloc_local([1], acc)
            lse_sum = T.alloc_local([1], acc)
            w = T.alloc_local([1], acc)
            T.clear(acc_o)
            T.clear(lse_sum)
            lse_max[0] = -T.infinity(acc)
            for k in T.serial(num_split):
                lse_max[0] = T.max(lse_max[0], glse[bz, by, k])
            for k in T.serial(num_split):
                lse_sum[0] += T.exp2(glse[bz, by, k] - lse_max[0])
            lse_sum[0] = T.log2(lse_sum[0]) + lse_max[0]
            for k in T.serial(num_split):
                for i in T.Parallel(dv):
                    part[i] = Opart[bz, by, k, i]
                w[0] = T.exp2(glse[bz, by, k] - lse_sum[0])
                for i in T.Parallel(dv):
                    acc_o[i] += part[i] * w[0]
            for i in T.Parallel(dv):
                Output[bz, by, i] = acc_o[i]

    if fp8:

        @T.prim_func
        def mla_fp8(Q: T.Tensor([batch, h_q, dv], dtype), Q_pe: T.Tensor([batch, h_q, dpe], dtype),
                    KV: T.Tensor([batch * max_seqlen_pad, h_kv, dv], kv_dtype),
                    K_pe: T.Tensor([batch * max_seqlen_pad, h_kv, dpe], kv_dtype),
                    block_table: T.Tensor([batch, pages], "int32"),
                    cache_seqlens: T.Tensor([batch], "int32"),
                    glse: T.Tensor([batch, h_q, num_split], acc),
                    Output_partial: T.Tensor([batch, h_q, num_split, dv], acc),
                    Output: T.Tensor([batch, h_q, dv], out_dtype),
                    KV_scale: T.Tensor([1], "float32")):
            split_kernel(Q, Q_pe, KV, K_pe, block_table, cache_seqlens, glse, Output_partial,
                         KV_scale)
            combine(glse, Output_partial, Output)

        return mla_fp8

    @T.prim_func
    def mla(Q: T.Tensor([batch, h_q, dv], dtype), Q_pe: T.Tensor([batch, h_q, dpe], dtype),
            KV: T.Tensor([batch * max_seqlen_pad, h_kv, dv], kv_dtype),
            K_pe: T.Tensor([batch * max_seqlen_pad, h_kv, dpe], kv_dtype),
            block_table: T.Tensor([batch, pages], "int32"),
            cache_seqlens: T.Tensor([batch], "int32"),
            glse: T.Tensor([batch, h_q, num_split], dtype),
            Output_partial: T.Tensor([batch, h_q, num_split, dv], dtype),
            Output: T.Tensor([batch, h_q, dv], out_dtype)):
        split_kernel(Q, Q_pe, KV, K_pe, block_table, cache_seqlens, glse, Output_partial, None)
        combine(glse, Output_partial, Output)

    return mla


def mla_decode_nopage(batch, heads, seqlen_kv, dim, pe_dim, block_N=64, block_H=64,
                      num_split=1, dtype="float16"):
    """examples/deepseek_mla/example_mla_decode.py:10-227: non-paged MLA decode, Q [batch,
    heads, dim], KV [batch, seqlen_kv, 1, dim], exp2 softmax with scale 1/sqrt(dim + pe_dim) *
    log2(e); main_split (num_split > 1: per-split partial outputs and log2 sum-exp in glse /
    Output_partial, then the LSE combine) or main_no_split. Output is parameter 6."""
    scale = (1.0 / (dim + pe_dim)) ** 0.5 * 1.44269504
    acc = "float"
    VB = min(block_H, heads)

    def attn(Q, Q_pe, KV, K_pe, Out, glse=None, Opart=None):
        grid = (batch, heads // VB) + ((num_split,) if glse is not None else ())
        with T.Kernel(*grid, threads=256) as ids:
            bx, by = ids[0], ids[1]
            bz = ids[2] if glse is not None else None
            q_s = T.alloc_shared([block_H, dim], dtype)
            s_s = T.alloc_shared([block_H, block_N], dtype)
            qpe_s = T.alloc_shared([block_H, pe_dim], dtype)
            kv_s = T.alloc_shared([block_N, dim], dtype)
            kpe_s = T.alloc_shared([block_N, pe_dim], dtype)
            o_s = T.alloc_shared([block_H, dim], dtype)
            s = T.alloc_fragment([block_H, block_N], acc)
            o = T.alloc_fragment([block_H, dim], acc)
            m = T.alloc_fragment([block_H], acc)
            m_prev = T.alloc_fragment([block_H], acc)
            alpha = T.alloc_fragment([block_H], acc)
            rsum = T.alloc_fragment([block_H], acc)
            l = T.alloc_fragment([block_H], acc)
            T.use_swizzle(10)
            T.copy(Q[bx, by * VB:(by + 1) * VB, :], q_s)
            T.copy(Q_pe[bx, by * VB:(by + 1) * VB, :], qpe_s)
            T.fill(o, 0)
            T.fill(l, 0)
            T.fill(m, -T.infinity(acc))
            per = seqlen_kv // num_split
            n_iter = T.ceildiv(per if glse is not None else seqlen_kv, block_N)
            for k in T.Pipelined(n_iter, num_stages=2):
                start = (per * bz if glse is not None else 0) + k * block_N
                T.copy(KV[bx, start:start + block_N, 0, :], kv_s)
                T.copy(K_pe[bx, start:start + block_N, 0, :], kpe_s)
                T.clear(s)
                T.gemm(q_s, kv_s, s, transpose_B=True, policy=T.GemmWarpPolicy.FullCol)
                T.gemm(qpe_s, kpe_s, s, transpose_B=True, policy=T.GemmWarpPolicy.FullCol)
                T.copy(m, m_prev)
                T.fill(m, -T.infinity(acc))
                T.reduce_max(s, m, dim=1, clear=False)
                for i in T.Parallel(block_H):
                    alpha[i] = T.exp2(m_prev[i] * scale - m[i] * scale)
                for i, j in T.Parallel(block_H, block_N):
                    s[i, j] = T.exp2(s[i, j] * scale - m[i] * scale)
                T.reduce_sum(s, rsum, dim=1)
                T.copy(s, s_s)
                for i in T.Parallel(block_H):
                    l[i] = l[i] * alpha[i] + rsum[i]
                for i, j in T.Parallel(block_H, dim):
                    o[i, j] *= alpha[i]
                T.gemm(s_s, kv_s, o, policy=T.GemmWarpPolicy.FullCol)
            for i, j in T.Parallel(block_H, dim):
                o[i, j] /= l[i]
            if glse is not None:
                for i in T.Parallel(block_H):
                    l[i] = T.log2(l[i]) + m[i] * scale
                T.copy(l, glse[bx, by * VB:(by + 1) * VB, bz])
                T.copy(o, o_s)
                T.copy(o_s, Opart[bx, by * VB:(by + 1) * VB, bz, :])
            else:
                T.copy(o, o_s)
                T.copy(o_s, Out[bx, by * VB:(by + 1) * VB, :])

    def combine(glse, Opart, Out):
        with T.Kernel(heads, batch, threads=128) as (by, bz):
            part = T.alloc_fragment([dim], dtype)
            acc_o = T.alloc_fragment([dim], acc)
            lse_max = T.alloc_local([1], acc)
            lse_sum = T.alloc_local([1], acc)
            w = T.alloc_local([1], acc)
            T.clear(lse_sum)
            T.clear(acc_o)
            lse_max[0] = -T.infinity(acc)
            for k in T.serial(num_split):
                lse_max[0] = T.max(lse_max[0], glse[bz, by, k])
            for k in T.serial(num_split):
                lse_sum[0] += T.exp2(glse[bz, by, k] - lse_max[0])
            lse_sum[0] = T.log2(lse_sum[0]) + lse_max[0]
            for k in T.serial(num_split):
                for i in T.Parallel(dim):
                    part[i] = Opart[bz, by, k, i]
                w[0] = T.exp2(glse[bz, by, k] - lse_sum[0])
                for i in T.Parallel(dim):
                    acc_o[i] += part[i] * w[0]
            for i in T.Parallel(dim):
                Out[bz, by, i] = acc_o[i]

    @T.prim_func
    def main(Q: T.Tensor([batch, heads, dim], dtype), Q_pe: T.Tensor([batch, heads, pe_dim], dtype),
             KV: T.Tensor([batch, seqlen_kv, 1, dim], dtype),
             K_pe: T.Tensor([batch, seqlen_kv, 1, pe_dim], dtype),
             glse: T.Tensor([batch, heads, num_split], dtype),
             Output_partial: T.Tensor([batch, heads, num_split, dim], dtype),
             Output: T.Tensor([batch, heads, dim], dtype)):
        if num_split > 1:
            attn(Q, Q_pe, KV, K_pe, None, glse, Output_partial)
            combine(glse, Output_partial, Output)
        else:
            attn(Q, Q_pe, KV, K_pe, Output)

    return main


def mla_decode_tpu(batch, heads, seqlen_kv, dim, pe_dim, block_N, block_H):
    """tpu_demo/ppl/deepseek_mla/mla_decode.py:9-121: the TPU program written with T.ppl_* ops.
    Q [batch, heads, 1, dim], KV [batch, seqlen_kv, 1, dim], fp16; scores scaled by
    1/sqrt(dim + pe_dim) with ppl_mul_C and exponentiated with ppl_exp2 (natural exp); P copied to
    an fp16 tile before the P @ KV gemm."""
    scale = (1.0 / (dim + pe_dim)) ** 0.5
    dtype, acc = "float16", "float"
    VB = min(block_H, heads)

    @T.prim_func
    def main(Q: T.Tensor([batch, heads, 1, dim], dtype),
             Q_pe: T.Tensor([batch, heads, 1, pe_dim], dtype),
             KV: T.Tensor([batch, seqlen_kv, 1, dim], dtype),
             K_pe: T.Tensor([batch, seqlen_kv, 1, pe_dim], dtype),
             Output: T.Tensor([batch, heads, 1, dim], dtype)):
        with T.Kernel(batch, T.ceildiv(heads, VB), is_cpu=True) as (bx, by):
            q_s = T.alloc_shared([VB, dim], dtype)
            qpe_s = T.alloc_shared([VB, pe_dim], dtype)
            kv_s = T.alloc_shared([block_N, dim], dtype)
            kpe_s = T.alloc_shared([block_N, pe_dim], dtype)
            p_s = T.alloc_shared([VB, block_N], dtype)
            o_s = T.alloc_shared([VB, dim], dtype)
            s = T.alloc_shared([VB, block_N], acc)
            s_pe = T.alloc_shared([VB, block_N], acc)
            o = T.alloc_shared([VB, dim], acc)
            m = T.alloc_shared([VB, 1], acc)
            m_prev = T.alloc_shared([VB, 1], acc)
            alpha = T.alloc_shared([VB, 1], acc)
            rsum = T.alloc_shared([VB, 1], acc)
            l = T.alloc_shared([VB, 1], acc)
            T.ppl_copy(Q[bx, by * VB:(by + 1) * VB, :, :], q_s)
            T.ppl_copy(Q_pe[bx, by * VB:(by + 1) * VB, :, :], qpe_s)
            T.ppl_fill(o, T.float32(0))
            T.ppl_fill(l, T.float32(0))
            T.ppl_fill(m, -T.infinity(acc))
            for k in T.Pipelined(T.ceildiv(seqlen_kv, block_N), num_stages=2):
                T.ppl_copy(KV[bx, k * block_N:(k + 1) * block_N, 0, :], kv_s)
                T.ppl_copy(K_pe[bx, k * block_N:(k + 1) * block_N, 0, :], kpe_s)
                T.ppl_clear(s)
                T.ppl_gemm(q_s, kv_s, s, transpose_B=True)
                T.ppl_clear(s_pe)
                T.ppl_gemm(qpe_s, kpe_s, s_pe, transpose_B=True)
                T.ppl_add(s, s, s_pe)
                T.ppl_copy(m, m_prev)
                T.ppl_fill(m, -T.infinity(acc))
                T.ppl_reduce_max(s, m, dim=1, clear=False)
                prev_scaled = T.alloc_shared([VB, 1], acc)
                curr_scaled = T.alloc_shared([VB, 1], acc)
                T.ppl_mul_C(prev_scaled, m_prev, scale)
                T.ppl_mul_C(curr_scaled, m, scale)
                T.ppl_subtract(alpha, prev_scaled, curr_scaled)
                T.ppl_exp2(alpha)
                m_scaled = T.alloc_shared([VB, 1], acc)
                T.ppl_mul_C(s, s, scale)
                T.ppl_mul_C(m_scaled, m, scale)
                T.ppl_subtract(s, s, m_scaled)
                T.ppl_exp2(s)
                T.ppl_reduce_sum(s, rsum, dim=1)
                T.ppl_copy(s, p_s)
                T.ppl_mul(l, l, alpha)
                T.ppl_add(l, l, rsum)
                T.ppl_mul(o, o, alpha)
                T.ppl_gemm(p_s, kv_s, o)
            T.ppl_div(o, o, l)
            T.ppl_copy(o, o_s)
            T.ppl_copy(o_s, Output[bx, by * VB:(by + 1) * VB, :, :])

    return main


def ppl_exp(M, N, block_M, block_N, dtype="float32"):
    """tpu_demo/ppl/test/exp.py:6-16 (and exp_bf16.py): in-place natural exp of [M, N]."""

    @T.prim_func
    def main(scores_scale: T.Tensor([M, N], dtype)):
        with T.Kernel(T.ceildiv(N, block_N), T.ceildiv(M, block_M), is_cpu=True) as (bx, by):
            t = T.alloc_shared([block_M, block_N], dtype)
            T.ppl_copy(scores_scale[by * block_M, bx * block_N], t)
            T.ppl_exp2(t, block_M, block_N, dtype)
            T.ppl_copy(t, scores_scale[by * block_M, bx * block_N])

    return main


def ppl_mul_rows(M, N, blk_m, dtype="float32"):
    """tpu_demo/ppl/test/mul_N_1.py:9-22: C = A * B with B [M, 1] broadcast along each row."""

    @T.prim_func
    def main(C: T.Tensor((M, N), dtype), A: T.Tensor((M, N), dtype), B: T.Tensor((M, 1), dtype)):
        with T.Kernel(T.ceildiv(M, blk_m), is_cpu=True) as (bx,):
            a_s = T.alloc_shared((blk_m, N), dtype)
            b_s = T.alloc_shared((blk_m, 1), dtype)
            T.ppl_copy(A[bx * blk_m:(bx + 1) * blk_m, :], a_s)
            T.ppl_copy(B[bx * blk_m:(bx + 1) * blk_m, 0], b_s)
            T.ppl_mul(a_s, a_s, b_s)
            T.ppl_copy(a_s, C[bx * blk_m:(bx + 1) * blk_m, :])

    return main


def ppl_scale_shift(M, N, blk_m, blk_n, dtype="float32", scale=1 / 8192, shift=1e-12):
    """tpu_demo/ppl/test/elementwise_c.py:9-22: B = A * (1/8192) + 1e-12 (ppl_mul_C, ppl_add_C)."""

    @T.prim_func
    def main(A: T.Tensor((M, N), dtype), B: T.Tensor((M, N), dtype)):
        with T.Kernel(T.ceildiv(M, blk_m), T.ceildiv(N, blk_n), is_cpu=True) as (bx, by):
            a_s = T.alloc_shared((blk_m, blk_n), dtype)
            T.ppl_copy(A[bx * blk_m, by * blk_n], a_s)
            T.ppl_mul_C(a_s, a_s, T.float32(scale))
            T.ppl_add_C(a_s, a_s, T.float32(shift))
            T.ppl_copy(a_s, B[bx * blk_m, by * blk_n])

    return main


def ppl_add(M, N, block_M, block_N, in_dtype="float32", out_dtype="float32"):
    """tpu_demo/ppl/elementwise_add_kernel/elementwise_add.py:9-35: C = A + B."""

    @T.prim_func
    def main(A: T.Tensor((M, N), in_dtype), B: T.Tensor((M, N), in_dtype),
             C: T.Tensor((M, N), out_dtype)):
        with T.Kernel(T.ceildiv(N, block_N), T.ceildiv(M, block_M), is_cpu=True) as (bx, by):
            a_s = T.alloc_shared((block_M, block_N), in_dtype)
            b_s = T.alloc_shared((block_M, block_N), in_dtype)
            c_s = T.alloc_shared((block_M, block_N), out_dtype)
            T.ppl_copy(A[by * block_M, bx * block_N], a_s)
            T.ppl_copy(B[by * block_M, bx * block_N], b_s)
            T.ppl_add(c_s, a_s, b_s)
            T.ppl_copy(c_s, C[by * block_M, bx * block_N])

    return main


def fill_tiles(M, N, block_M, block_N, dtype="float16", accum_dtype="float", value=0.0):
    """tpu_demo/ppl/matmul.py:9-23: every block_M x block_N tile of A [M, N] is filled with a
    constant in an accum_dtype tile and copied out (cast to dtype). The demo calls it with
    symbolic extents, matmul(T.symbolic("m"), T.symbolic("n"), 128, 128, 2) (:26)."""

    @T.prim_func
    def main(A: T.Tensor((M, N), dtype)):
        with T.Kernel(T.ceildiv(N, block_N), T.ceildiv(M, block_M), is_cpu=True) as (bx, by):
            a_s = T.alloc_shared((block_M, block_N), accum_dtype)
            T.ppl_fill(a_s, T.float32(value))
            T.copy(a_s, A[by * block_M, bx * block_N])

    return main


def add_symbolic(block_M, block_N, dtype="float32"):
    """tpu_demo/ppl/elementwise_add_kernel/elementwise_add.py:9-35 over symbolic extents m, n
    (T.symbolic, reference tilelang/language/__init__.py:85-86): C = A + B for any [m, n]."""
    return ppl_add(T.symbolic("m"), T.symbolic("n"), block_M, block_N, dtype, dtype)
