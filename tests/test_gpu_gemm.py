"""GPU parity: GEMM through ``tilelang.compile`` against the fp32-accumulate oracle.

Tolerance atol=rtol=1e-2 (tpu_demo/matmul/tpu_test_matmul_fp16.py:56); a result within one
output rounding of the fp32 oracle is also required for all but a 1e-4 fraction of elements
(accumulation order differs from the CPU's).
"""
import pytest
import torch

import tilelang
from tilelang.jit.adapter.mi355x import ops
from tilelang.testing import programs, workloads
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_matmul_demo_program_tpu_convention():
    """tpu_demo/matmul/tpu_test_matmul_fp16.py flow: 64^3, CPU tensors, C written in place."""
    k = tilelang.compile(programs.matmul(64, 64, 64, 32, 32, 32), out_idx=-1, target="tpu")
    g = torch.Generator().manual_seed(11)
    a = torch.randn(64, 64, generator=g).half()
    b = torch.randn(64, 64, generator=g).half()
    c = torch.zeros(64, 64).half()
    assert k(a, b, c) == 0
    torch_assert_close(c, ref.matmul_ref(a, b), atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("M,N,K,dtype", [
    (4096, 4096, 4096, torch.float16),
    (4096, 4096, 4096, torch.bfloat16),
    (16, 14336, 4096, torch.float16),
    (16, 14336, 4096, torch.bfloat16),
    (300, 264, 136, torch.float16),
    (1, 8, 8, torch.float16),
    (7, 1000, 520, torch.bfloat16),
    (513, 777, 1000, torch.float16),
])
def test_gemm_shapes(M, N, K, dtype):
    w = workloads.gemm(M, N, K, dtype=dtype, seed=12)
    dn = "float16" if dtype == torch.float16 else "bfloat16"
    k = tilelang.compile(programs.matmul(M, N, K, 128, 128, 64, dn, "float16"), out_idx=-1)
    c = k(w.tensors["a"].to(DEV), w.tensors["b"].to(DEV))
    exp = ref.matmul_ref(w.tensors["a"], w.tensors["b"])
    torch_assert_close(c.cpu(), exp, atol=1e-2, rtol=1e-2)
    torch_assert_close(c.cpu(), exp, atol=1e-3, rtol=1e-3, max_mismatched_ratio=1e-4)


@pytest.mark.parametrize("M,N,K", [(256, 512, 256), (16, 4096, 1024), (100, 300, 200)])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_gemm_trans_b_and_out_dtypes(M, N, K, out):
    g = torch.Generator().manual_seed(13)
    a = (torch.rand(M, K, generator=g) * 2 - 1).half()
    bt = (torch.rand(N, K, generator=g) * 2 - 1).half()
    c = torch.empty(M, N, dtype=out, device=DEV)
    ops.gemm(a.to(DEV), bt.to(DEV), c, trans_b=True)
    exp = ref.matmul_ref(a, bt, out_dtype=out, trans_b=True)
    torch_assert_close(c.cpu(), exp, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("M,N,K", [(5, 100, 96), (16, 1000, 520), (3, 4104, 4096)])
def test_gemm_skinny_nonfinite_column_stays_in_its_column(M, N, K):
    """The skinny kernel reads whole 64-column strips of B; in the last, ragged strip the columns
    past N hold the next row's leading values. A NaN / inf column 0 of B must reach column 0 of C
    only: every other column matches the oracle."""
    g = torch.Generator().manual_seed(M + N + K)
    a = (torch.rand(M, K, generator=g) * 2 - 1).half()
    b = (torch.rand(K, N, generator=g) * 2 - 1).half()
    b[:, 0] = float("nan")
    b[1::2, 0] = float("inf")
    c = torch.empty(M, N, dtype=torch.float16, device=DEV)
    ops.gemm(a.to(DEV), b.to(DEV), c)
    c = c.cpu()
    assert not torch.isfinite(c[:, 0]).any()
    torch_assert_close(c[:, 1:], ref.matmul_ref(a, b)[:, 1:], atol=1e-2, rtol=1e-2)


def test_gemm_skinny_split_repeatable():
    """M <= 16 with row-major B splits K over several workgroups per column strip; the partial
    tiles are summed in split order by whichever workgroup arrives last, and the arrival counters
    are left at zero: reruns are bitwise equal, also after calls of other shapes in between."""
    g = torch.Generator().manual_seed(21)
    a = (torch.rand(16, 4096, generator=g) * 2 - 1).half().to(DEV)
    b = (torch.rand(4096, 4096, generator=g) * 2 - 1).half().to(DEV)
    c0 = torch.empty(16, 4096, dtype=torch.float16, device=DEV)
    ops.gemm(a, b, c0)
    torch_assert_close(c0.cpu(), ref.matmul_ref(a.cpu(), b.cpu()), atol=1e-2, rtol=1e-2)
    for m, n, k in [(3, 1000, 520), (16, 512, 4096), (16, 4096, 4096)]:
        x = torch.randn(m, k, device=DEV).half()
        y = torch.randn(k, n, device=DEV).half()
        ops.gemm(x, y, torch.empty(m, n, dtype=torch.float16, device=DEV))
        c = torch.empty_like(c0)
        ops.gemm(a, b, c)
        assert torch.equal(c, c0)


@pytest.mark.parametrize("M,N,K", [(16, 4096, 14336), (5, 1000, 2056), (1, 64, 8192),
                                   (16, 520, 4104)])
def test_gemm_skinny_bt_split(M, N, K):
    """M <= 16 with B^T and few 64-column strips splits K over several workgroups per strip
    (one per CU in all); the partial tiles meet in split order: parity with the oracle, and
    reruns (with other split calls in between) are bitwise equal."""
    g = torch.Generator().manual_seed(M + N + K)
    a = (torch.rand(M, K, generator=g) * 2 - 1).half()
    b = (torch.rand(N, K, generator=g) * 2 - 1).half()
    c0 = torch.empty(M, N, dtype=torch.float16, device=DEV)
    ops.gemm(a.to(DEV), b.to(DEV), c0, trans_b=True)
    torch_assert_close(c0.cpu(), ref.matmul_ref(a, b.t().contiguous()), atol=1e-2, rtol=1e-2)
    x = torch.randn(3, 1000, device=DEV).half()
    ops.gemm(x, torch.randn(200, 1000, device=DEV).half(),
             torch.empty(3, 200, dtype=torch.float16, device=DEV), trans_b=True)
    c1 = torch.empty_like(c0)
    ops.gemm(a.to(DEV), b.to(DEV), c1, trans_b=True)
    assert torch.equal(c1, c0)


def test_gemm_skinny_concurrent_streams():
    """Each stream owns one workspace slot of the split skinny kernel (4 per device); further
    streams take the unsplit kernel. Six streams run skinny GEMMs at the same time, twice over,
    and every result matches the oracle."""
    g = torch.Generator().manual_seed(22)
    shapes = [(16, 4096, 4096), (8, 6144, 2048), (16, 2048, 8192), (1, 4096, 4096),
              (5, 3000, 1000), (16, 4096, 4096)]
    ins = [((torch.rand(m, k, generator=g) * 2 - 1).half(),
            (torch.rand(k, n, generator=g) * 2 - 1).half()) for m, n, k in shapes]
    dev_ins = [(x.to(DEV), y.to(DEV)) for x, y in ins]
    outs = [torch.empty(m, n, dtype=torch.float16, device=DEV) for m, n, _ in shapes]
    streams = [torch.cuda.Stream() for _ in shapes]
    torch.cuda.synchronize()
    for _ in range(2):
        for (x, y), c, st in zip(dev_ins, outs, streams):
            with torch.cuda.stream(st):
                ops.gemm(x, y, c)
    torch.cuda.synchronize()
    for (x, y), c in zip(ins, outs):
        torch_assert_close(c.cpu(), ref.matmul_ref(x, y), atol=1e-2, rtol=1e-2)


def test_gemm_skinny_split_graph_replays():
    """A skinny GEMM captured in a HIP graph (no memset node: the split kernel's arrival counters
    are reset by the kernel) gives, on every replay, the bits of the same call run eagerly on
    the capture stream, with eager skinny GEMMs of other shapes run between the replays. (The
    capture stream owns a workspace slot, or takes the unsplit kernel when earlier streams of
    the process hold all slots; the eager call on that stream takes the same path.)"""
    g = torch.Generator().manual_seed(23)
    a_h = (torch.rand(16, 4096, generator=g) * 2 - 1).half()
    b_h = (torch.rand(4096, 6144, generator=g) * 2 - 1).half()
    a, b = a_h.to(DEV), b_h.to(DEV)
    c = torch.zeros(16, 6144, dtype=torch.float16, device=DEV)
    ref_c = torch.empty_like(c)
    graph, side = torch.cuda.CUDAGraph(), torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.gemm(a, b, ref_c)
        with torch.cuda.graph(graph, stream=side):
            ops.gemm(a, b, c)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    torch_assert_close(ref_c.cpu(), ref.matmul_ref(a_h, b_h), atol=1e-2, rtol=1e-2)
    x = torch.randn(8, 2048, device=DEV).half()
    y = torch.randn(2048, 3000, device=DEV).half()
    for _ in range(3):
        c.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(c, ref_c)
        ops.gemm(x, y, torch.empty(8, 3000, dtype=torch.float16, device=DEV))
        torch.cuda.synchronize()


def test_gemm_generic_path_odd_k():
    """K not a multiple of 8 takes the scalar fallback kernel."""
    g = torch.Generator().manual_seed(14)
    a = torch.randn(33, 45, generator=g).half()
    b = torch.randn(45, 27, generator=g).half()
    c = torch.empty(33, 27, dtype=torch.float16, device=DEV)
    ops.gemm(a.to(DEV), b.to(DEV), c)
    torch_assert_close(c.cpu(), ref.matmul_ref(a, b), atol=1e-2, rtol=1e-2)


def test_gemm_identity_and_consistency():
    """A @ I == A exactly (fp32 accumulation of exact products), and reruns are bitwise equal."""
    a = torch.randn(512, 512, generator=torch.Generator().manual_seed(15)).half().to(DEV)
    eye = torch.eye(512, dtype=torch.float16, device=DEV)
    c = torch.empty_like(a)
    ops.gemm(a, eye, c)
    assert torch.equal(c, a)
    k = tilelang.compile(programs.matmul(1024, 1024, 1024, 128, 128, 64), out_idx=-1)
    k.get_profiler().assert_consistent(repeat=3)
