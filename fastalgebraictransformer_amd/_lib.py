"""ctypes binding of libkat.so (C ABI declared in include/kat.h).

The library is loaded lazily, after ``torch`` (so its libamdhip64.so.7
dependency binds to the HIP runtime PyTorch already loaded). There is no
fallback: if the library is missing or fails to load, every GPU call raises.
"""

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkat.so")

_lock = threading.Lock()
_lib = None

_DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.float64: 3}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_INT = ctypes.c_int
_SZ = ctypes.c_size_t
_I64P = ctypes.POINTER(ctypes.c_int64)

_SIGNATURES = {
    "kat_version": ([], _INT),
    "kat_last_error": ([], ctypes.c_char_p),
    "kat_rsoftmax_fwd": ([_P, _P, _I64, _I64, _I64, _I64, _F, _INT, _P], _INT),
    "kat_rsoftmax_bwd": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _INT, _P], _INT),
    "kat_rswiglu_fwd": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _INT, _P], _INT),
    "kat_rswiglu_bwd": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _INT, _P],
                        _INT),
    "kat_men_fwd": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F, _INT, _INT, _P], _INT),
    "kat_men_bwd_workspace_size": ([_I64, _I64, _INT], _SZ),
    "kat_men_bwd": ([_P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I64, _I64, _F, _INT,
                     _INT, _P], _INT),
    "kat_add_men_fwd": ([_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _INT,
                         _INT, _INT, _INT, _P], _INT),
    "kat_add_men_bwd": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I64, _I64,
                         _I64, _I64, _F, _INT, _INT, _INT, _INT, _P], _INT),
    "kat_attn_fwd": ([_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64P, _I64P, _F, _F, _INT,
                      _INT, _P], _INT),
    "kat_attn_bwd_workspace_size": ([_I64, _I64, _I64, _I64, _INT], _SZ),
    "kat_attn_bwd": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I64,
                      _I64P, _I64P, _F, _F, _INT, _INT, _P], _INT),
    "kat_attn_fwd_masked": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64P,
                             _I64P, _F, _F, _INT, _INT, _P], _INT),
    "kat_attn_bwd_masked_workspace_size": ([_I64, _I64, _I64, _I64, _INT, _INT], _SZ),
    "kat_attn_bwd_masked": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _SZ, _I64,
                             _I64, _I64, _I64, _I64P, _I64P, _F, _F, _INT, _INT, _P], _INT),
    "kat_attn_decode_workspace_size": ([_I64, _I64, _I64, _I64, _INT], _SZ),
    "kat_attn_decode": ([_P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I64, _I64P, _F,
                         _F, _INT, _P], _INT),
    "kat_attn_decode_noalloc": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64P, _F, _F,
                                 _INT, _P], _INT),
    "kat_probe_mfma_bf16": ([_P, _INT, _INT, ctypes.POINTER(ctypes.c_double), _P], _INT),
    "kat_probe_mfma_bf16_random": ([_P, _INT, _INT, ctypes.POINTER(ctypes.c_double), _P], _INT),
}

EXPORTED = tuple(_SIGNATURES)


def load():
    """Load libkat.so once and declare the C signatures; raise if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is not built; run `python -m fastalgebraictransformer_amd.build` "
                    "(or __graft_entry__.build()) first")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (args, res) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = res
            _lib = lib
    return _lib


def dtype_code(t):
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32/bfloat16/float16/float64")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(t):
    """The current torch stream of t's device as a hipStream_t (the raw-pointer
    query, where torch has it, skips building a Stream object on every launch)."""
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(t.device.index))
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def check(rc, name):
    if rc != 0:
        msg = load().kat_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {rc}): {msg}")


def i64_array(values):
    arr = (ctypes.c_int64 * len(values))(*[int(x) for x in values])
    return arr


def rows2d(t):
    """View ``t`` as [rows, cols] over its last dim without copying when the
    layout allows (unit last-dim stride, collapsible leading dims, rows that do
    not overlap); otherwise return a contiguous copy. Returns (t2d, ld)."""
    if t.dim() == 0:
        t = t.reshape(1)
    cols = t.shape[-1]
    if cols == 1 or t.stride(-1) == 1:
        try:
            t2 = t.view(-1, cols)
        except RuntimeError:
            t2 = None
        if t2 is not None:
            ld = t2.stride(0) if t2.shape[0] > 1 else cols
            if ld >= cols and (cols == 1 or t2.stride(1) == 1):
                return t2, ld
    t2 = t.contiguous().view(-1, cols)
    return t2, cols
