"""GPU timing (reference tilelang/profiler/bench.py:9-102, re-done for MI355X).

The reference times with CUDA events and zeroes a 256 MB buffer before each rep to flush L2.
MI355X has a 256 MB Infinity Cache (MALL) behind its L2s, so 256 MB does not evict it; the flush
buffer here is 512 MiB. Events are recorded on the current stream, which is the stream the
kernels are launched on.
"""
from typing import Callable, List, Literal, Optional, Union

import torch

FLUSH_BYTES = 512 << 20
_flush = {}


def flush_buffer(device=None) -> torch.Tensor:
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    buf = _flush.get(dev)
    if buf is None:
        buf = torch.empty(FLUSH_BYTES // 4, dtype=torch.int32, device=dev)
        _flush[dev] = buf
    return buf


def do_bench(fn: Callable, warmup: float = 25, rep: float = 100, _n_warmup: int = 0,
             _n_repeat: int = 0, grad_to_none=None, quantiles: Optional[List[float]] = None,
             fast_flush: bool = True, flush: bool = True,
             return_mode: Literal["min", "max", "mean", "median"] = "mean"
             ) -> Union[float, List[float]]:
    """Milliseconds per call of ``fn`` (mean by default), each rep after a cache flush."""
    assert return_mode in ("min", "max", "mean", "median")
    fn()
    torch.cuda.synchronize()
    cache = flush_buffer() if flush else None
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(5):
        if cache is not None:
            cache.zero_()
        fn()
    e.record()
    torch.cuda.synchronize()
    est = max(s.elapsed_time(e) / 5, 1e-3)
    n_warmup = _n_warmup if _n_warmup > 0 else max(1, int(warmup / est))
    n_repeat = _n_repeat if _n_repeat > 0 else max(1, int(rep / est))
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n_repeat)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n_repeat)]
    for _ in range(n_warmup):
        fn()
    for i in range(n_repeat):
        if grad_to_none is not None:
            for x in grad_to_none:
                x.grad = None
        if cache is not None:
            cache.zero_()
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    times = torch.tensor([a.elapsed_time(b) for a, b in zip(starts, ends)], dtype=torch.float)
    if quantiles is not None:
        r = torch.quantile(times, torch.tensor(quantiles, dtype=torch.float)).tolist()
        return r[0] if len(r) == 1 else r
    return getattr(torch, return_mode)(times).item()
