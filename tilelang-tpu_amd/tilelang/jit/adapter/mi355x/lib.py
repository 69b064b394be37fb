"""ctypes binding of libtlmi355x.so (include/tlmi355x.h).

The reference binds its generated ``main.so`` the same way: ``ctypes.CDLL`` then
``tilelang_tpu_run.argtypes = [POINTER(c_void_p)]; restype = c_int``
(tilelang/jit/adapter/cython/adapter.py:211-216, libgen.py:33-36). Here the library is built
once (tilelang-tpu_amd/build_lib.py) and every operator family has its own typed entry point.
A missing library raises: there is no CPU fallback behind this adapter.
"""
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
_DEFAULT = os.path.normpath(os.path.join(_HERE, "..", "..", "..", "lib", "libtlmi355x.so"))

# enum tlm_dtype
F16, BF16, F32, F8E4M3, I32, F8E5M2, U32 = 0, 1, 2, 3, 4, 5, 6
REDUCE_MAX, REDUCE_SUM = 0, 1

_lock = threading.Lock()
_lib = None

c_void_p, c_int, c_int64, c_float, c_size_t = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64,
                                               ctypes.c_float, ctypes.c_size_t)

_SIGNATURES = {
    "tlm_version": ([], c_int),
    "tlm_init": ([c_int], c_int),
    "tlm_last_error": ([], ctypes.c_char_p),
    "tlm_num_cus": ([], c_int),
    "tlm_rmsnorm": ([c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_float, c_int, c_void_p],
                    c_int),
    "tlm_swiglu": ([c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p], c_int),
    "tlm_rope": ([c_void_p] * 6 + [c_int64] * 4 + [c_int, c_void_p], c_int),
    "tlm_gemm": ([c_void_p] * 3 + [c_int64] * 3 + [c_int] * 3 + [c_void_p], c_int),
    "tlm_gemm_fp8": ([c_void_p] * 3 + [c_int64] * 3 + [c_int] * 3 + [c_void_p], c_int),
    "tlm_flash_attn_fwd": ([c_void_p] * 4 + [c_int64] * 4 + [c_int, c_float, c_int, c_void_p],
                           c_int),
    "tlm_flash_attn_fwd_ex": ([c_void_p] * 4 + [c_int64] * 5 +
                              [c_int, c_float, c_int, c_int, c_void_p], c_int),
    "tlm_flash_attn_varlen_fwd": ([c_void_p] * 6 + [c_int64] * 7 +
                                  [c_int, c_float, c_int, c_int, c_void_p], c_int),
    "tlm_flash_attn_bhsd_fwd": ([c_void_p] * 4 + [c_int64] * 6 +
                                [c_int, c_float, c_int, c_int, c_void_p], c_int),
    "tlm_flash_attn_splitkv_workspace_bytes": ([c_int64] * 5 + [c_int], c_size_t),
    "tlm_flash_attn_splitkv_fwd": ([c_void_p] * 7 + [c_size_t] + [c_int64] * 6 +
                                   [c_int, c_float, c_int, c_void_p], c_int),
    "tlm_cast": ([c_void_p, c_int, c_void_p, c_int, c_int64, c_void_p], c_int),
    "tlm_sigmoid": ([c_void_p, c_void_p, c_int64, c_int, c_void_p], c_int),
    "tlm_gather_rows": ([c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p],
                        c_int),
    "tlm_topk": ([c_void_p, c_int64, c_int64, c_int, c_int, c_void_p, c_void_p, c_void_p], c_int),
    "tlm_row_reduce": ([c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_int, c_void_p],
                       c_int),
    "tlm_mla_decode": ([c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64,
                        c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t] +
                       [c_int64] * 6 + [c_int, c_float, c_void_p, c_int, c_int, c_int, c_void_p], c_int),
    "tlm_mla_decode_ex": ([c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                           c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t] +
                          [c_int64] * 6 + [c_int, c_float, c_void_p, c_int, c_int, c_int,
                                           c_void_p, c_void_p, c_int64, c_int, c_void_p], c_int),
    "tlm_mla_workspace_bytes": ([c_int64, c_int64, c_int64, c_int], c_size_t),
    "tlm_mla_decode_noalloc": ([c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                c_int64, c_int64, c_void_p, c_void_p, c_void_p] +
                               [c_int64] * 6 + [c_int, c_float, c_void_p, c_int, c_int, c_int,
                                                c_void_p], c_int),
    "tlm_mla_scratch_bytes": ([], c_size_t),
    "tlm_paged_gather": ([c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
                          c_int64, c_int64, c_int64, c_void_p], c_int),
    "tlm_elementwise": ([ctypes.POINTER(c_void_p), ctypes.POINTER(c_int),
                         ctypes.POINTER(c_int), c_int, ctypes.POINTER(c_void_p),
                         ctypes.POINTER(c_int), c_int, ctypes.POINTER(ctypes.c_int32), c_int,
                         ctypes.POINTER(c_float), c_int, c_int64, c_int64, c_void_p], c_int),
    "tlm_kv_append_fp8": ([c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p, c_void_p,
                           c_int64, c_int64, c_void_p] + [c_int64] * 5 + [c_void_p, c_void_p],
                          c_int),
}

EXPORTED = tuple(_SIGNATURES)

# enum tlm_ew_op / tlm_ew_bcast (include/tlmi355x.h)
EW_LOAD, EW_CONST, EW_ADD, EW_SUB, EW_MUL, EW_DIV, EW_EXP, EW_RSQRT, EW_SIGMOID, EW_ROUND, \
    EW_STORE = range(11)
EW_FULL, EW_ROW, EW_COL, EW_SCALAR = range(4)
EW_SLOTS, EW_MAX_IN, EW_MAX_OUT, EW_MAX_CODE, EW_MAX_CONST = 8, 8, 4, 64, 16


def library_path() -> str:
    return os.environ.get("TLMI355X_LIB", _DEFAULT)


def load():
    """Load (once) and type the library. Raises RuntimeError if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"libtlmi355x.so not found at {path}: build it with "
                f"`python tilelang-tpu_amd/build_lib.py` (or __graft_entry__.build()). "
                f"The mi355x target has no CPU fallback.")
        lib = ctypes.CDLL(path)
        for name, (argtypes, restype) in _SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = lib
        return lib


class TLMError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


def check(fn_name: str, rc: int):
    if rc != 0:
        msg = load().tlm_last_error().decode("utf-8", "replace")
        raise TLMError(fn_name, rc, msg)
    return rc


def call(fn_name: str, *args):
    """Call ``fn_name`` and raise :class:`TLMError` on a nonzero status."""
    lib = load()
    return check(fn_name, getattr(lib, fn_name)(*args))


_inited = set()


def ensure_device(index: int):
    if index in _inited:
        return
    call("tlm_init", index)
    _inited.add(index)
