"""CPU tests of the drop-in boundary: tracing, recognition, JITKernel surface, argument
validation (modelled on cython_wrapper.pyx:76-79, 130-150 and base.py:20-44 of the reference)."""
import math

import pytest
import torch

import tilelang
import tilelang.language as T
from tilelang.jit.adapter.base import legalize_result_idx
from tilelang.jit.adapter.mi355x import UnsupportedProgram
from tilelang.jit.adapter.mi355x.recognize import recognize
from tilelang.testing import programs


def test_recognize_each_family():
    cases = [
        (programs.rms_norm(128, 128, 32), "rmsnorm", dict(eps=1e-12, cols=128, w=None)),
        (programs.rms_norm(64, 4096, 1, eps=1e-6, with_weight=True), "rmsnorm",
         dict(eps=1e-6, w=1, y=2)),
        (programs.matmul(64, 96, 32, 32, 32, 32), "gemm", dict(M=64, N=96, K=32, trans_b=False)),
        (programs.matmul(64, 96, 32, 32, 32, 32, trans_b=True), "gemm", dict(trans_b=True)),
        (programs.rope(64, 16, 128, 64), "rope", dict(tokens=128, heads_q=1, dim=64)),
        (programs.rope_qk(10, 4, 2, 128), "rope", dict(heads_q=4, heads_k=2, tokens=10)),
        (programs.swi_glu(32, 32, 64, 64), "swiglu", dict(gate=0, up=1, out=2, n=4096)),
        (programs.flashattn(1, 2, 256, 128, True), "flashattn", dict(causal=True, S=256)),
        (programs.flashattn(1, 2, 256, 64, False), "flashattn", dict(causal=False, D=64)),
        (programs.mla_decode(2, 128, 1, 256, 512, 64, 64, 64, 4, 64), "mla",
         dict(num_split=4, page=64, max_pages=4, kv_dtype="float16")),
        (programs.mla_decode(2, 128, 1, 256, 512, 64, 64, 64, 1, 32, dtype="bfloat16",
                             kv_dtype="float8_e4m3"), "mla",
         dict(num_split=1, page=32, kv_scale=9, kv_dtype="float8_e4m3")),
    ]
    for prog, fam, attrs in cases:
        k = tilelang.compile(prog, out_idx=-1 if fam != "mla" else [8], target="mi355x")
        assert k.plan.family == fam, (prog, k.plan)
        for key, val in attrs.items():
            assert k.plan.attrs[key] == val, (fam, key, k.plan.attrs[key], val)
        assert fam in k.get_kernel_source()


def test_softmax_scales_are_read_from_the_program():
    fa = tilelang.compile(programs.flashattn(1, 2, 256, 128, True), out_idx=-1)
    assert math.isclose(fa.plan.attrs["sm_scale"], 1 / math.sqrt(128), rel_tol=1e-12)
    mla = tilelang.compile(programs.mla_decode(2, 128, 1, 256, 512, 64, 64, 64, 2, 64),
                           out_idx=[8])
    assert math.isclose(mla.plan.attrs["sm_scale"], 1 / math.sqrt(576), rel_tol=1e-9)


def test_reference_fa_demo_style_copy_alias():
    """tpu_test_flashattn_bf16.py:11 rebinds T.copy = T.ppl_copy before defining the program."""
    saved = T.copy
    try:
        T.copy = T.ppl_copy
        k = tilelang.compile(programs.flashattn(1, 2, 128, 128, False), out_idx=-1, target="tpu")
        assert k.plan.family == "flashattn"
    finally:
        T.copy = saved


def test_symbolic_branch_is_traced():
    """`if kr == 0:` on a loop variable (example_mla_decode_paged.py:77) records a branch."""

    @T.prim_func
    def prog(A: T.Tensor((64, 64), "float16"), B: T.Tensor((64, 64), "float16")):
        with T.Kernel(2, threads=64) as bx:
            s = T.alloc_shared((32, 64), "float16")
            for kr in T.Pipelined(4, num_stages=2):
                if kr == 0:
                    T.ppl_copy(A[bx * 32, 0], s)
            T.ppl_copy(s, B[bx * 32, 0])

    names = [op.name for op in prog.ops]
    assert "branch" in names and names.count("ppl_copy") == 2
    with pytest.raises(UnsupportedProgram):
        tilelang.compile(prog, out_idx=-1)


def test_unsupported_program_rejected():

    @T.prim_func
    def mix(A: T.Tensor((64, 64), "float32"), B: T.Tensor((64, 1), "float32")):
        with T.Kernel(1, is_cpu=True) as (bx,):
            a = T.alloc_shared((64, 64), "float32")
            m = T.alloc_shared((64, 1), "float32")
            T.ppl_copy(A[0, 0], a)
            T.ppl_exp2(a)  # an exponential feeding a row max: no kernel family
            T.ppl_reduce_max(a, m, dim=1)
            T.ppl_copy(m, B[0, 0])

    with pytest.raises(UnsupportedProgram, match="no gfx950 kernel"):
        tilelang.compile(mix, out_idx=-1)


def test_elementwise_programs_are_recognised():
    """The stand-alone elementwise demos compile into register programs; an rsqrt alone is
    one too; a tile copy that does not cover its tensor is rejected."""
    k = tilelang.compile(programs.ppl_mul_rows(8192, 8192, 64), out_idx=[0])
    a = k.plan.attrs
    assert k.plan.family == "elementwise" and a["inputs"] == [1, 2] and a["bcast"] == [0, 1]
    assert (a["rows"], a["cols"]) == (8192, 8192)
    k = tilelang.compile(programs.ppl_scale_shift(16, 4, 4, 2), out_idx=-1)
    assert k.plan.attrs["consts"] == [1 / 8192, 1e-12]

    @T.prim_func
    def rs(A: T.Tensor((64, 64), "float32"), B: T.Tensor((64, 64), "float32")):
        with T.Kernel(1, is_cpu=True) as (bx,):
            a = T.alloc_shared((64, 64), "float32")
            T.ppl_copy(A[0, 0], a)
            T.ppl_rsqrt(a, a)
            T.ppl_copy(a, B[0, 0])

    assert tilelang.compile(rs, out_idx=-1).plan.family == "elementwise"

    @T.prim_func
    def part(A: T.Tensor((64, 64), "float32"), B: T.Tensor((64, 64), "float32")):
        with T.Kernel(1, is_cpu=True) as (bx,):
            a = T.alloc_shared((32, 64), "float32")  # one 32-row tile of a 64-row tensor
            T.ppl_copy(A[0, 0], a)
            T.ppl_rsqrt(a, a)
            T.ppl_copy(a, B[0, 0])

    with pytest.raises(UnsupportedProgram, match="grid"):
        tilelang.compile(part, out_idx=-1)


def test_unsupported_variants_have_clear_errors():
    # fp32 matrix tiles (no cast to 16-bit tiles before ppl_gemm): no fp32-operand kernel
    with pytest.raises(UnsupportedProgram, match="tiles"):
        tilelang.compile(programs.matmul(64, 64, 64, 32, 32, 32, dtype="float32",
                                         out_dtype="float32"), out_idx=-1)
    # fp32 attention tiles are the all-fp32 program tpu_demo/ppl/flashattn/fa_fp32.py
    k = tilelang.compile(programs.flashattn(1, 2, 4, 8, False, 2, 2, dtype="float32"),
                         out_idx=-1)
    assert k.plan.attrs["dtype"] == "float32" and k.plan.attrs["operand_dtype"] is None
    # fp32 attention tiles with a 16-bit output are not a program of the reference
    with pytest.raises(UnsupportedProgram):
        tilelang.compile(_fa_fp32_tiles_bf16_out(), out_idx=-1)


def _fa_fp32_tiles_bf16_out():
    import copy
    from tilelang.language import ir
    base = programs.flashattn(1, 2, 4, 8, False, 2, 2, dtype="float32")
    bad = copy.copy(base)
    o = base.params[3]
    bad.params = list(base.params[:3]) + [ir.Buffer(o.name, o.shape, "bfloat16", "global")]
    return bad


@pytest.mark.parametrize("name,prog,attrs", [
    ("rmsnorm_fp32.py", lambda: programs.rms_norm(128, 512, 32, dtype="float32"),
     dict(dtype="float32", cols=512, eps=1e-12)),
    ("rmsnorm_splitk_fp16.py", lambda: programs.rms_norm_splitk(512, 512, 32, 32),
     dict(dtype="float16", rows=512, cols=512)),
    ("rmsnorm_splitk_bf16.py", lambda: programs.rms_norm_splitk(512, 512, 32, 32, "bfloat16"),
     dict(dtype="bfloat16")),
    ("rmsnorm_splitk_fp32.py", lambda: programs.rms_norm_splitk(512, 512, 32, 32, "float32"),
     dict(dtype="float32")),
    ("tpu_test_matmul_fp32.py", lambda: programs.matmul(64, 64, 64, 32, 32, 32, "float32",
                                                        "float32", operand_dtype="float16"),
     dict(in_dtype="float32", out_dtype="float32", operand_dtype="float16")),
    ("tpu_test_rope_fp32.py", lambda: programs.rope(64, 16, 128, 64, dtype="float32"),
     dict(dtype="float32", dim=64, tokens=128)),
    ("tpu_test_rope_fp16.py", lambda: programs.rope(64, 16, 128, 64, dtype="float16"),
     dict(dtype="float16")),
    ("tpu_test_swiglu_fp32.py", lambda: programs.swi_glu(32, 32, 1024, 1024, dtype="float32"),
     dict(dtype="float32", n=1024 * 1024)),
    ("tpu_test_flashattn_fp16.py", lambda: programs.flashattn(1, 2, 4, 8, False, 2, 2,
                                                              dtype="float16"),
     dict(dtype="float16", D=8, S=4, operand_dtype=None)),
    ("tpu_test_flashattn_fp32.py", lambda: programs.flashattn(1, 2, 4, 8, False, 2, 2,
                                                              dtype="float32",
                                                              gemm_dtype="float16"),
     dict(dtype="float32", D=8, operand_dtype="float16")),
    ("tpu_test_sigmoid_fp32.py", lambda: programs.sigmoid(32, 32, 1024, 1024),
     dict(dtype="float32", n=1024 * 1024)),
    ("tpu_test_gather_fp32.py", lambda: programs.gather(128, 64, 8),
     dict(rows=128, hidden=64, n=8, dtype="float32")),
    ("tpu_test_topk_fp32.py", lambda: programs.topk(1024, 8),
     dict(k=8, descending=True, length=1024)),
    ("tpu_test_reduce_max.py", lambda: programs.row_reduce(64, 64, 32, 64, "max"),
     dict(op="max", rows=64, cols=64)),
    ("tpu_test_reduce_sum.py", lambda: programs.row_reduce(64, 64, 32, 64, "sum"),
     dict(op="sum", in_dtype="float16")),
])
def test_demo_variants_recognised(name, prog, attrs):
    """The remaining tpu_demo programs (fp32 / fp16 twins, split-K RMSNorm) map to a family."""
    plan = recognize(prog())
    for k, v in attrs.items():
        assert plan.attrs[k] == v, (name, k, plan.attrs[k])


def test_bhsd_flashattn_program():
    """examples/flash_attention/example_mha_fwd_bhsd.py: head-major tensors, @T.macro helpers with
    T.SharedBuffer / T.FragmentBuffer annotations, seq_q != seq_kv; causal only at equal
    lengths (the example's mask and loop bound disagree otherwise)."""
    k = tilelang.compile(programs.flashattn_bhsd(1, 1, 256, 256, 64, False), out_idx=[3])
    a = k.plan.attrs
    assert k.plan.family == "flashattn" and a["layout"] == "bhsd" and not a["causal"]
    assert (a["B"], a["H"], a["H_kv"], a["S"], a["S_kv"], a["D"]) == (1, 1, 1, 256, 256, 64)
    assert math.isclose(a["sm_scale"], 1 / math.sqrt(64), rel_tol=1e-9)
    p = recognize(programs.flashattn_bhsd(2, 8, 300, 1000, 128, False, dtype="bfloat16"))
    assert (p.attrs["S"], p.attrs["S_kv"], p.attrs["H"], p.attrs["dtype"]) == (300, 1000, 8,
                                                                               "bfloat16")
    c = recognize(programs.flashattn_bhsd(2, 4, 512, 512, 128, True))
    assert c.attrs["causal"] and c.attrs["layout"] == "bhsd"
    with pytest.raises(UnsupportedProgram, match="seq_q"):
        recognize(programs.flashattn_bhsd(1, 4, 128, 512, 64, True))
    # sequence-major programs keep their layout
    assert "layout" not in recognize(programs.flashattn_gqa(1, 4, 256, 64, False)).attrs


def test_varlen_flashattn_program():
    """examples/flash_attention/example_mha_fwd_varlen.py: a scalar T.int32 parameter
    (max_seqlen_q), int32 cu_seqlens, element-wise tile fills; only the non-causal form maps."""
    k = tilelang.compile(programs.flashattn_varlen(2, 500, 510, 16, 32), out_idx=-1)
    a = k.plan.attrs
    assert k.plan.family == "flashattn" and a["varlen"] and not a["causal"]
    assert (a["q"], a["k"], a["v"], a["cu_q"], a["cu_k"], a["max_q"], a["o"]) == (0, 1, 2, 3, 4,
                                                                                   5, 6)
    assert (a["B"], a["H"], a["H_kv"], a["D"]) == (2, 16, 16, 32)
    assert math.isclose(a["sm_scale"], 1 / math.sqrt(32), rel_tol=1e-9)
    assert k.params[5].is_scalar() and k.out_idx == [6]
    gq = recognize(programs.flashattn_varlen(3, 700, 650, 8, 128, groups=4, dtype="bfloat16"))
    assert (gq.attrs["H_kv"], gq.attrs["total_k"]) == (2, 650)
    with pytest.raises(UnsupportedProgram, match="causal"):
        recognize(programs.flashattn_varlen(2, 500, 510, 16, 32, is_causal=True))
    # scalar arguments are Python ints; tensors are validated as before
    q = torch.zeros(500, 16, 32).half()
    kv = torch.zeros(510, 16, 32).half()
    cu = torch.zeros(3, dtype=torch.int32)
    with pytest.raises(ValueError, match="scalar"):
        k(q, kv, kv, cu, cu, torch.tensor(256))
    with pytest.raises(ValueError, match="scalar"):
        k(q, kv, kv, cu, cu, 256.0)
    with pytest.raises(ValueError, match="Expected 7 arguments"):
        k(q, kv, kv, cu, cu)
    # the profiler's random supply has nothing to give a scalar (as the reference's supply)
    from tilelang.utils.tensor import TensorSupplyType, get_tensor_supply
    with pytest.raises(ValueError, match="must have a shape"):
        get_tensor_supply(TensorSupplyType.Auto)(k.params[5])


def test_scalar_params_rejected():
    with pytest.raises(TypeError, match="T.Tensor"):

        @T.prim_func
        def bad(A: T.Tensor((4,), "float16"), n: int):
            pass


def test_targets_and_modes():
    prog = programs.swi_glu(32, 32, 64, 64)
    for t in ("auto", "tpu", "mi355x", "hip"):
        assert tilelang.compile(prog, out_idx=-1, target=t).target == "mi355x"
    with pytest.raises(ValueError, match="not supported"):
        tilelang.compile(prog, out_idx=-1, target="cuda")
    with pytest.raises(AssertionError, match="mode"):
        tilelang.compile(prog, out_idx=-1, mode="fpga")
    with pytest.raises(AssertionError, match="backend"):
        tilelang.compile(prog, out_idx=-1, execution_backend="tvm")
    assert tilelang.compile(prog, out_idx=-1, mode="cmodel").mode == "cmodel"


def test_out_idx_legalisation():
    assert legalize_result_idx(-1, 4) == [3]
    assert legalize_result_idx([0, -1], 4) == [0, 3]
    assert legalize_result_idx(None, 4) == []
    for bad in (4, -5, [4], "x"):
        with pytest.raises(ValueError):
            legalize_result_idx(bad, 4)
    k = tilelang.compile(programs.rope_qk(4, 2, 2, 64), out_idx=None)
    assert k.out_idx == [4, 5]  # the recogniser knows which parameters are written


def test_kernel_surface():
    k = tilelang.compile(programs.matmul(64, 64, 64, 32, 32, 32), out_idx=-1, target="tpu")
    assert [p.dtype for p in k.params] == [torch.float16] * 3
    assert [p.shape for p in k.params] == [[64, 64]] * 3
    assert k.out_idx == [2]
    assert callable(k.func) and k.func is k.adapter.func
    prof = k.get_profiler()
    assert prof.result_idx == [2]


def test_argument_validation_before_device():
    k = tilelang.compile(programs.swi_glu(32, 32, 64, 64), out_idx=-1)
    a = torch.randn(64, 64).bfloat16()
    with pytest.raises(ValueError, match="Expected 3 arguments"):
        k(a)
    with pytest.raises(ValueError, match="dtype mismatch"):
        k(a.float(), a)
    with pytest.raises(ValueError, match="shape mismatch"):
        k(torch.randn(32, 64).bfloat16(), a)
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="no CPU fallback"):
            k(a, a)


def _gemm_with_epilogue(M=64, N=64, K=64, blk=32, kind="scale"):
    """ppl GEMM programs whose result is not A @ B: a scaled accumulator, a bias tile added
    before the copy-out, a bias parameter loaded into the accumulator, an unused extra tensor,
    or an accumulator filled with 1."""
    @T.prim_func
    def main(A: T.Tensor((M, K), "float16"), B: T.Tensor((K, N), "float16"),
             Bias: T.Tensor((M, N), "float32"), C: T.Tensor((M, N), "float16")):
        with T.Kernel(T.ceildiv(N, blk), T.ceildiv(M, blk), is_cpu=True) as (bx, by):
            a_s = T.alloc_shared((blk, blk), "float16")
            b_s = T.alloc_shared((blk, blk), "float16")
            acc = T.alloc_shared((blk, blk), "float32")
            bias = T.alloc_shared((blk, blk), "float32")
            c_s = T.alloc_shared((blk, blk), "float16")
            if kind == "bias_init":
                T.ppl_copy(Bias[by * blk, bx * blk], acc)
            else:
                T.ppl_fill(acc, T.float32(1.0 if kind == "fill_one" else 0.0))
            for k in T.Pipelined(T.ceildiv(K, blk), num_stages=2):
                T.ppl_copy(A[by * blk, k * blk], a_s)
                T.ppl_copy(B[k * blk, bx * blk], b_s)
                T.ppl_gemm(a_s, b_s, acc)
            if kind == "scale":
                T.ppl_mul_C(acc, acc, T.float32(2.0))
            if kind == "bias_add":
                T.ppl_copy(Bias[by * blk, bx * blk], bias)
                T.ppl_add(acc, acc, bias)
            T.ppl_copy(acc, c_s)
            T.ppl_copy(c_s, C[by * blk, bx * blk])

    return main


@pytest.mark.parametrize("kind", ["scale", "bias_add", "bias_init", "unused", "fill_one"])
def test_gemm_with_epilogue_or_extra_tensor_is_rejected(kind):
    with pytest.raises(UnsupportedProgram):
        recognize(_gemm_with_epilogue(kind=kind))


def test_gemm_element_epilogue_is_rejected_but_2xacc_fold_is_not():
    """The fp8 2xAcc fold (acc2[i, j] += acc[i, j]) is the only element store a GEMM may have;
    a scaling store in the same place is rejected."""
    assert recognize(programs.matmul_fp8(256, 256, 256, two_acc=True)).family == "gemm"

    @T.prim_func
    def main(A: T.Tensor((64, 64), "float16"), B: T.Tensor((64, 64), "float16"),
             C: T.Tensor((64, 64), "float32")):
        with T.Kernel(2, 2, threads=128) as (bx, by):
            a_s = T.alloc_shared((32, 64), "float16")
            b_s = T.alloc_shared((64, 32), "float16")
            acc = T.alloc_fragment((32, 32), "float")
            T.clear(acc)
            T.copy(A[by * 32, 0], a_s)
            T.copy(B[0, bx * 32], b_s)
            T.gemm(a_s, b_s, acc)
            for i, j in T.Parallel(32, 32):
                acc[i, j] = acc[i, j] * 0.5
            T.copy(acc, C[by * 32, bx * 32])

    with pytest.raises(UnsupportedProgram):
        recognize(main)


def test_flashattn_with_extra_parameter_is_rejected():
    """A tensor parameter that the matched attention pattern never touches is an error (the
    kernel would silently leave it unwritten or ignore it)."""
    import copy
    from tilelang.language import ir
    base = programs.flashattn(1, 2, 256, 128, False)
    assert recognize(base).family == "flashattn"
    extra = copy.copy(base)
    extra.params = list(base.params[:3]) + [ir.Buffer("Extra", (1, 256, 2, 128), "bfloat16",
                                                      "global")] + list(base.params[3:])
    with pytest.raises(UnsupportedProgram, match="Extra"):
        recognize(extra)


def test_nonpaged_mla_programs_are_recognised():
    """example_mla_decode.py (split / no-split) and the TPU program mla_decode.py (ppl ops,
    natural exp, [batch, heads, 1, dim]) map to the MLA family in non-paged mode, with the
    program's own softmax scale; a 3-gemm program without int32 parameters is no longer sent to
    the SwiGLU matcher."""
    k = tilelang.compile(programs.mla_decode_nopage(2, 128, 512, 512, 64, num_split=4),
                         out_idx=[6])
    a = k.plan.attrs
    assert k.plan.family == "mla" and not a["paged"] and a["seqlen_kv"] == 512
    assert a["num_split"] == 4 and (a["glse"], a["o_partial"], a["o"]) == (4, 5, 6)
    assert math.isclose(a["sm_scale"], 1 / math.sqrt(576), rel_tol=1e-9)
    t = tilelang.compile(programs.mla_decode_tpu(4, 8, 512, 32, 4, 4, 4), out_idx=-1)
    a = t.plan.attrs
    assert t.plan.family == "mla" and not a["paged"] and (a["dv"], a["dpe"], a["Hq"]) == (32, 4, 8)
    assert math.isclose(a["sm_scale"], 1 / 6, rel_tol=1e-12)
    assert t.plan.out_idx == [4]


def test_splitkv_inference_program_recognised():
    """example_mha_inference.py: recognised as sequence-major attention with seq_q != seq_kv;
    splits that drop or overlap keys and the program's causal form are rejected."""
    k = tilelang.compile(programs.mha_inference(1, 32, 128, 8192, 128), out_idx=[5])
    a = k.plan.attrs
    assert k.plan.family == "flashattn" and a["layout"] == "bshd_kv"
    assert (a["S"], a["S_kv"], a["num_split"], a["o"]) == (128, 8192, 4, 5)
    assert abs(a["sm_scale"] - 128 ** -0.5) < 1e-6
    with pytest.raises(UnsupportedProgram, match="whole 64-key tiles"):
        tilelang.compile(programs.mha_inference(1, 32, 128, 8000, 128), out_idx=[5])
    with pytest.raises(UnsupportedProgram, match="causal"):
        tilelang.compile(programs.mha_inference(1, 32, 128, 8192, 128, is_causal=True),
                         out_idx=[5])


def test_mlp_program_recognised_with_whole_blocks_only():
    k = tilelang.compile(programs.deepseek_mlp(64, 256, 512, 128, 256, 512), out_idx=[0])
    a = k.plan.attrs
    assert k.plan.family == "mlp" and (a["x"], a["wg"], a["wu"], a["wd"], a["out"]) == (1, 2, 3, 4, 0)
    assert (a["M"], a["hidden"], a["inter"]) == (128, 256, 512)
    with pytest.raises(UnsupportedProgram, match="whole blocks"):
        tilelang.compile(programs.deepseek_mlp(8, 8, 8, 16, 16, 16), out_idx=[0])


def test_fp32_mlp_program_recognised():
    """tpu_demo/ppl/mlp/mlp_fp32.py: fp32 parameters, bf16 gemm tiles; whole blocks only."""
    k = tilelang.compile(programs.deepseek_mlp_fp32(16, 16, 16, 16, 16, 16), out_idx=[0])
    a = k.plan.attrs
    assert k.plan.family == "mlp" and a["dtype"] == "float32"
    assert a["operand_dtype"] == "bfloat16"
    with pytest.raises(UnsupportedProgram, match="whole blocks"):
        tilelang.compile(programs.deepseek_mlp_fp32(8, 8, 8, 16, 16, 16), out_idx=[0])


def test_elementwise_tile_at_another_grid_position_is_rejected():
    """An input tile taken at the transposed grid position of the output tile reads other
    elements than the ones it is stored to: not an elementwise program."""

    @T.prim_func
    def swapped(A: T.Tensor((64, 64), "float32"), B: T.Tensor((64, 64), "float32")):
        with T.Kernel(2, 2, is_cpu=True) as (bx, by):
            a = T.alloc_shared((32, 32), "float32")
            T.ppl_copy(A[by * 32, bx * 32], a)
            T.ppl_rsqrt(a, a)
            T.ppl_copy(a, B[bx * 32, by * 32])

    with pytest.raises(UnsupportedProgram, match="grid position"):
        tilelang.compile(swapped, out_idx=-1)

    @T.prim_func
    def same(A: T.Tensor((64, 64), "float32"), B: T.Tensor((64, 64), "float32")):
        with T.Kernel(2, 2, is_cpu=True) as (bx, by):
            a = T.alloc_shared((32, 32), "float32")
            T.ppl_copy(A[by * 32, bx * 32], a)
            T.ppl_rsqrt(a, a)
            T.ppl_copy(a, B[by * 32, bx * 32])

    assert tilelang.compile(same, out_idx=-1).plan.family == "elementwise"


def test_elementwise_reload_after_store_is_rejected():
    """A copy from a parameter after the program stored to it would read the stored values;
    the register program loads each input once, so such a program is rejected."""

    @T.prim_func
    def reload(A: T.Tensor((64, 64), "float32"), B: T.Tensor((64, 64), "float32")):
        with T.Kernel(1, is_cpu=True) as (bx,):
            a = T.alloc_shared((64, 64), "float32")
            b = T.alloc_shared((64, 64), "float32")
            T.ppl_copy(A[0, 0], a)
            T.ppl_add(a, a, a)
            T.ppl_copy(a, A[0, 0])
            T.ppl_copy(A[0, 0], b)
            T.ppl_add(b, b, b)
            T.ppl_copy(b, B[0, 0])

    with pytest.raises(UnsupportedProgram, match="after the program stores"):
        tilelang.compile(reload, out_idx=-1)


def test_symbolic_extents_specialise_per_call():
    """T.symbolic (reference tilelang/language/__init__.py:85-86): the demo's fill program
    (tpu_demo/ppl/matmul.py:26) compiles with symbolic m, n; each call binds them from the
    argument shapes and recognises the specialised program (rows / cols from the binding)."""
    m, n = T.symbolic("m"), T.symbolic("n")
    prog = programs.fill_tiles(m, n, 128, 128)
    assert prog.symbolic_vars() == ["m", "n"]
    k = tilelang.compile(prog, out_idx=-1)
    assert k.plan.family == "elementwise" and k.adapter.dynamic
    spec = prog.specialize({"m": 300, "n": 520})
    assert tuple(spec.params[0].shape) == (300, 520)
    assert [ir_const(e) for e in spec.kernels[0].extents] == [5, 3]  # ceil(520/128), ceil(300/128)
    plan = k.adapter._plan_for({"m": 300, "n": 520})
    assert (plan.attrs["rows"], plan.attrs["cols"]) == (300, 520)
    assert plan.attrs["consts"] == [0.0] and not plan.attrs["inputs"]
    # the same binding is recognised once
    assert k.adapter._plan_for({"m": 300, "n": 520}) is plan
    # the elementwise add over symbolic m, n: shapes must agree under the binding (checked
    # before any device work, so this runs without a GPU)
    add = tilelang.compile(programs.add_symbolic(64, 64), out_idx=-1)
    with pytest.raises(ValueError, match="mismatch"):
        add(torch.zeros(4, 5), torch.zeros(4, 6))
    with pytest.raises(ValueError, match="mismatch"):
        add(torch.zeros(4, 5), torch.zeros(3, 5))


def test_symbolic_extent_checked_after_every_binding():
    """An extent that depends on a variable bound by a later argument (2 * m in the first
    parameter, m bound by the second) is still compared with the argument's size."""
    from tilelang.language import ir
    add = tilelang.compile(programs.add_symbolic(64, 64), out_idx=-1)
    ad = add.adapter
    m = next(s for s in ad.params[1].shape if isinstance(s, ir.Var) and s.name == "m")
    env = {}
    ad._check(1, torch.zeros(4, 5), env)
    assert env == {"m": 4, "n": 5}
    ad.params[0].shape = [m * 2, ad.params[0].shape[1]]
    try:
        ad._check_bound(0, torch.zeros(8, 5), env)
        with pytest.raises(ValueError, match="mismatch"):
            ad._check_bound(0, torch.zeros(4, 5), env)
        with pytest.raises(ValueError, match="not bound"):
            ad._check_bound(0, torch.zeros(8, 5), {"n": 5})
    finally:
        ad.params[0].shape = list(ad.params[1].shape)


def ir_const(e):
    from tilelang.language import ir
    return ir.const_value(e)


def test_symbolic_program_still_fails_at_compile_time():
    """A symbolic program that fits no kernel family is rejected by tilelang.compile, at the
    trial binding, not at the first call."""
    m = T.symbolic("m")

    @T.prim_func
    def mix(A: T.Tensor((m, 64), "float32"), B: T.Tensor((m, 1), "float32")):
        with T.Kernel(T.ceildiv(m, 64), is_cpu=True) as (bx,):
            a = T.alloc_shared((64, 64), "float32")
            r = T.alloc_shared((64, 1), "float32")
            T.ppl_copy(A[bx * 64, 0], a)
            T.ppl_exp2(a)
            T.ppl_reduce_max(a, r, dim=1)
            T.ppl_copy(r, B[bx * 64, 0])

    with pytest.raises(UnsupportedProgram):
        tilelang.compile(mix, out_idx=-1)


# ------------------------------------------------------------------------------------------------
# The dedicated families take parameter roles from the data flow and compile only the expression
# their kernel computes (anything else is rejected or goes to the general elementwise program).


def test_rope_output_first_program_roles():
    """tpu_demo/ppl/rope/rope_bf16.py:8-13 puts the output first."""
    k = tilelang.compile(programs.rope(64, 16, 128, 64, out_first=True), out_idx=[0])
    a = k.plan.attrs
    assert (a["q"], a["cos"], a["sin"], a["q_out"], a["k"]) == (1, 2, 3, 0, None)
    assert k.out_idx == [0]


def _rope_variant(e2_kind="neg_x", cos_pos=None, C=128, W=64, Bc=64, Bw=16):
    dt = "bfloat16"

    @T.prim_func
    def main(X: T.Tensor((C, W), dt), CO: T.Tensor((C, W), dt), SI: T.Tensor((C, W), dt),
             O: T.Tensor((C, W), dt)):
        with T.Kernel(T.ceildiv(C, Bc), T.ceildiv(W, Bw), is_cpu=True) as (bx, by):
            x, c, s = (T.alloc_shared((Bc, Bw), dt) for _ in range(3))
            T.ppl_copy(X[bx * Bc, by * Bw], x)
            T.ppl_copy(CO[cos_pos(bx, by) if cos_pos else (bx * Bc, by * Bw)], c)
            T.ppl_copy(SI[bx * Bc, by * Bw], s)
            xc, xs, xn, e2, o = (T.alloc_shared((Bc, Bw), dt) for _ in range(5))
            T.ppl_mul(xc, x, c)
            T.ppl_mul(xs, x, s)
            if e2_kind == "neg_x":       # the demo: (-x) * sin
                T.ppl_mul_C(xn, x, -1.0)
                T.ppl_mul(e2, xn, s)
            elif e2_kind == "neg_prod":  # -(x * sin)
                T.ppl_mul_C(e2, xs, -1.0)
            elif e2_kind == "no_neg":    # x * sin: not a rotation
                T.ppl_mul(e2, x, s)
            elif e2_kind == "cos":       # (-x) * cos: the tables mixed up
                T.ppl_mul_C(xn, x, -1.0)
                T.ppl_mul(e2, xn, c)
            T.ppl_rope_add(o, xc, e2, xc, xs)
            T.ppl_copy(o, O[bx * Bc, by * Bw])

    return main


def test_rope_operand_forms():
    for kind in ("neg_x", "neg_prod"):
        a = recognize(_rope_variant(kind)).attrs
        assert (a["q"], a["cos"], a["sin"], a["q_out"]) == (0, 1, 2, 3)
    for kind in ("no_neg", "cos"):
        with pytest.raises(UnsupportedProgram, match="ppl_rope_add"):
            recognize(_rope_variant(kind))


def test_rope_tables_at_another_tile_rejected():
    # cos taken at the transposed tile position of a square grid
    prog = _rope_variant(cos_pos=lambda bx, by: (by * 64, bx * 64), C=128, W=128, Bc=64, Bw=64)
    with pytest.raises(UnsupportedProgram, match="grid position"):
        recognize(prog)


def _swiglu_variant(with_gate_factor):
    C = W = 64
    dt = "float32"

    @T.prim_func
    def main(G: T.Tensor((C, W), dt), U: T.Tensor((C, W), dt), O: T.Tensor((C, W), dt)):
        with T.Kernel(T.ceildiv(C, 32), T.ceildiv(W, 32), is_cpu=True) as (bx, by):
            g, u, e, ones, den, sig, out = (T.alloc_shared((32, 32), dt) for _ in range(7))
            T.ppl_fill(ones, T.float32(1.0))
            T.ppl_copy(G[bx * 32, by * 32], g)
            T.ppl_copy(U[bx * 32, by * 32], u)
            T.ppl_mul_C(e, g, T.float32(-1.0))
            T.ppl_exp2(e)
            T.ppl_add(den, e, ones)
            T.ppl_div(sig, g if with_gate_factor else ones, den)
            T.ppl_mul(out, sig, u)
            T.ppl_copy(out, O[bx * 32, by * 32])

    return main


def test_swiglu_expression_checked():
    p = recognize(_swiglu_variant(True))
    assert p.family == "swiglu" and (p.attrs["gate"], p.attrs["up"]) == (0, 1)
    # up * sigmoid(gate) is not SwiGLU: the general elementwise program computes it as written
    assert recognize(_swiglu_variant(False)).family == "elementwise"


def _rmsnorm_variant(kind):
    M, N, dt = 64, 128, "float32"

    def body(A, Wt, B):
        with T.Kernel(T.ceildiv(M, 32), is_cpu=True) as (bx,):
            x = T.alloc_shared((32, N), dt)
            sq = T.alloc_shared((32, N), dt)
            ss = T.alloc_shared((32, 1), dt)
            T.ppl_copy(A[bx * 32, 0], x)
            T.ppl_mul(sq, x, x)
            T.ppl_reduce_sum(sq, ss, dim=1)
            T.ppl_mul_C(ss, ss, T.float32(1.0 / N))
            T.ppl_add_C(ss, ss, T.float32(1e-6))
            T.ppl_rsqrt(ss, ss)
            if kind != "no_x":
                T.ppl_mul(x, x, ss)
            else:
                T.ppl_mul(x, sq, ss)  # x * x scaled: not RMSNorm
            if kind == "weight":
                w = T.alloc_shared((1, N), dt)
                T.ppl_copy(Wt[0], w)
                T.ppl_mul(x, x, w)
            T.ppl_copy(x, B[bx * 32, 0])

    if kind == "plain" or kind == "no_x":
        @T.prim_func
        def main(A: T.Tensor((M, N), dt), B: T.Tensor((M, N), dt)):
            body(A, None, B)
    else:
        @T.prim_func
        def main(A: T.Tensor((M, N), dt), Wt: T.Tensor((N,), dt), B: T.Tensor((M, N), dt)):
            body(A, Wt, B)
    return main


def test_rmsnorm_expression_checked():
    assert recognize(_rmsnorm_variant("plain")).attrs["w"] is None
    assert recognize(_rmsnorm_variant("weight")).attrs["w"] == 1
    # a weight parameter the program never applies is not multiplied in by the kernel either
    with pytest.raises(UnsupportedProgram, match="stored value"):
        recognize(_rmsnorm_variant("unused_weight"))
    with pytest.raises(UnsupportedProgram, match="stored value"):
        recognize(_rmsnorm_variant("no_x"))


def test_sigmoid_expression_checked():
    C = W = 64

    @T.prim_func
    def twice(G_in: T.Tensor((C, W), "float32"), G_out: T.Tensor((C, W), "float32")):
        with T.Kernel(T.ceildiv(C, 32), T.ceildiv(W, 32), is_cpu=True) as (bx, by):
            x, y = T.alloc_shared((32, 32), "float32"), T.alloc_shared((32, 32), "float32")
            T.ppl_copy(G_in[bx * 32, by * 32], x)
            T.ppl_sigmoid(y, x)
            T.ppl_mul_C(y, y, T.float32(2.0))
            T.ppl_copy(y, G_out[bx * 32, by * 32])

    assert recognize(programs.sigmoid(32, 32, C, W)).family == "sigmoid"
    assert recognize(twice).family == "elementwise"


def test_region_of_an_access_with_a_slice():
    """Point indices of an access that has a slice span one element; an access of point indices
    only takes the tile's extents on its trailing dims (tilelang/language/copy.py:40-62)."""
    from tilelang.language import ir
    buf = ir.Buffer("b", (10, 4, 128), "bfloat16", "global")
    st, ex = buf[3:7, 2, :].region((4, 128))
    assert [int(ir.const_value(e)) for e in ex] == [4, 1, 128]
    st, ex = buf[3, 2, 0].region((4, 128))
    assert [int(ir.const_value(e)) for e in ex] == [1, 4, 128]


def _gemm_variant(kind, M=64, N=64, K=128, BM=32, BN=32, BK=32):
    dt = "float16"

    @T.prim_func
    def main(A: T.Tensor((M, K), dt), B: T.Tensor((K, N), dt), C: T.Tensor((M, N), dt)):
        with T.Kernel(T.ceildiv(N, BN), T.ceildiv(M, BM), is_cpu=True) as (bx, by):
            a_s = T.alloc_shared((BM, BK), dt)
            b_s = T.alloc_shared((BK, BN), dt)
            acc = T.alloc_shared((BM, BN), "float32")
            c_s = T.alloc_shared((BM, BN), dt)
            if kind != "clear_inside":
                T.ppl_fill(acc, T.float32(0))
            nk = T.ceildiv(K, BK) - (1 if kind == "short_k" else 0)
            for k in T.Pipelined(nk, num_stages=2):
                if kind == "clear_inside":
                    T.ppl_fill(acc, T.float32(0))
                ra = bx if kind == "a_rows_by_bx" else by
                T.ppl_copy(A[ra * BM, k * BK], a_s)
                T.ppl_copy(B[k * BK, bx * BN], b_s)
                T.ppl_gemm(a_s, b_s, acc)
            T.ppl_copy(acc, c_s)
            T.ppl_copy(c_s, C[by * BM, bx * BN])

    return main


def test_gemm_tiles_and_k_coverage_checked():
    assert recognize(_gemm_variant("ok")).attrs["K"] == 128
    for kind, msg in (("short_k", "all of K"), ("a_rows_by_bx", "all of K"),
                      ("clear_inside", "cleared inside")):
        with pytest.raises(UnsupportedProgram, match=msg):
            recognize(_gemm_variant(kind))
    # 2xAcc with an odd k-tile count: the fold every second tile never takes the last one
    with pytest.raises(UnsupportedProgram, match="last k tile"):
        recognize(programs.matmul_fp8(256, 256, 192, two_acc=True))


def _reduce_variant(N, BN, clear=True, looped=False):
    M, BM = 64, 32

    @T.prim_func
    def main(X: T.Tensor((M, N), "float16"), Y: T.Tensor((M, 1), "float16")):
        with T.Kernel(1, T.ceildiv(M, BM), is_cpu=True) as (bx, by):
            xs = T.alloc_shared((BM, BN), "float16")
            ys = T.alloc_shared((BM, 1), "float16")
            if looped:
                T.ppl_fill(ys, T.float16(-65504.0))
                for k in T.serial(T.ceildiv(N, BN)):
                    T.ppl_copy(X[by * BM, k * BN], xs)
                    T.ppl_reduce_max(xs, ys, 1, False)
            else:
                T.ppl_copy(X[by * BM, 0], xs)
                T.ppl_reduce_max(xs, ys, 1, clear)
            T.ppl_copy(ys, Y[by * BM, 0])

    return main


def test_row_reduce_whole_rows():
    """tpu_test_reduce_max.py reduces one whole-row tile; a narrower tile reduces part of the
    row, a reduction without clear also takes the output's contents."""
    assert recognize(_reduce_variant(64, 64)).family == "row_reduce"
    with pytest.raises(UnsupportedProgram, match="whole rows"):
        recognize(_reduce_variant(128, 64))
    with pytest.raises(UnsupportedProgram, match="clearing reduction"):
        recognize(_reduce_variant(64, 64, clear=False))
    with pytest.raises(UnsupportedProgram, match="clearing reduction"):
        recognize(_reduce_variant(128, 64, looped=True))


def test_rmsnorm_whole_rows():
    """A row tile narrower than the row, or a looped row sum that is not accumulated."""
    M, N = 64, 128

    def prog(kind):
        @T.prim_func
        def main(A: T.Tensor((M, N), "float32"), B: T.Tensor((M, N), "float32")):
            with T.Kernel(T.ceildiv(M, 32), is_cpu=True) as (bx,):
                w = 64 if kind != "ok" else N
                x = T.alloc_shared((32, w), "float32")
                sq = T.alloc_shared((32, w), "float32")
                ss = T.alloc_shared((32, 1), "float32")
                if kind == "overwrite":
                    for k in T.serial(N // w):
                        T.ppl_copy(A[bx * 32, k * w], x)
                        T.ppl_mul(sq, x, x)
                        T.ppl_reduce_sum(sq, ss, dim=1)
                else:
                    T.ppl_copy(A[bx * 32, 0], x)
                    T.ppl_mul(sq, x, x)
                    T.ppl_reduce_sum(sq, ss, dim=1)
                T.ppl_mul_C(ss, ss, T.float32(1.0 / N))
                T.ppl_add_C(ss, ss, T.float32(1e-6))
                T.ppl_rsqrt(ss, ss)
                if kind == "overwrite":
                    for k in T.serial(N // w):
                        T.ppl_copy(A[bx * 32, k * w], x)
                        T.ppl_mul(x, x, ss)
                        T.ppl_copy(x, B[bx * 32, k * w])
                else:
                    T.ppl_mul(x, x, ss)
                    T.ppl_copy(x, B[bx * 32, 0])
        return main

    assert recognize(prog("ok")).family == "rmsnorm"
    with pytest.raises(UnsupportedProgram, match="whole rows"):
        recognize(prog("narrow"))
    with pytest.raises(UnsupportedProgram, match="accumulate"):
        recognize(prog("overwrite"))


def test_flashattn_visits_every_key_block():
    assert recognize(programs.flashattn(1, 2, 256, 64, False, 64, 64)).family == "flashattn"
    with pytest.raises(UnsupportedProgram, match="every key"):
        recognize(programs.flashattn(1, 2, 256, 64, False, 64, 64, kv_blocks=3))


def test_mlp_expression_checked():
    """The down projection must multiply up * silu(gate); silu(gate) * gate is another MLP."""
    M, Hd, I, dt, acc = 16, 64, 128, "bfloat16", "float32"

    def prog(second):
        @T.prim_func
        def main(output: T.Tensor((M, Hd), dt), x: T.Tensor((M, Hd), dt),
                 gate_weight: T.Tensor((I, Hd), dt), up_weight: T.Tensor((I, Hd), dt),
                 down_weight: T.Tensor((Hd, I), dt)):
            with T.Kernel(1, 1, 1, is_cpu=True) as (bx, by, bz):
                xb = T.alloc_shared((M, Hd), dt)
                wg, wu = T.alloc_shared((I, Hd), dt), T.alloc_shared((I, Hd), dt)
                wd = T.alloc_shared((Hd, I), dt)
                g16, u16 = T.alloc_shared((M, I), dt), T.alloc_shared((M, I), dt)
                d16, h16 = T.alloc_shared((M, Hd), dt), T.alloc_shared((M, I), dt)
                g32, u32, s32, h32, neg, ones, den = (T.alloc_shared((M, I), acc)
                                                      for _ in range(7))
                T.ppl_fill(ones, T.float32(1.0))
                T.ppl_copy(x[0:M, 0:Hd], xb)
                T.ppl_copy(gate_weight[0:I, 0:Hd], wg)
                T.ppl_copy(up_weight[0:I, 0:Hd], wu)
                T.ppl_copy(down_weight[0:Hd, 0:I], wd)
                T.ppl_gemm(xb, wg, g16, transpose_B=True)
                T.ppl_copy(g16, g32)
                T.ppl_mul_C(neg, g32, T.float32(-1.0))
                T.ppl_exp2(neg)
                T.ppl_add(den, neg, ones)
                T.ppl_div(s32, g32, den)
                T.ppl_gemm(xb, wu, u16, transpose_B=True)
                T.ppl_copy(u16, u32)
                T.ppl_mul(h32, s32, u32 if second == "up" else g32)
                T.ppl_copy(h32, h16)
                T.ppl_gemm(h16, wd, d16, transpose_B=True)
                T.ppl_copy(d16, output[0:M, 0:Hd])
        return main

    assert recognize(prog("up")).family == "mlp"
    with pytest.raises(UnsupportedProgram, match="silu"):
        recognize(prog("gate"))
