"""Loads ``libgdn.so`` (the HIP kernels behind ``include/gdn.h``) with ctypes
and binds its C ABI.

There is no fallback: if the library is missing, or if it would bind a
second HIP runtime next to torch's, loading raises. Tensors cross the
boundary as raw device pointers; work goes to torch's current stream.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgdn.so")
ABI_VERSION = 16

GDN_F32, GDN_BF16, GDN_F16 = 0, 1, 2
GDN_EINVAL, GDN_EUNSUPPORTED = -1, -2

_DTYPE_CODES = {torch.float32: GDN_F32, torch.bfloat16: GDN_BF16, torch.float16: GDN_F16}

_c_void_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_float = ctypes.c_float
_c_i64_p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); must match include/gdn.h
_SIGNATURES = {
    "gdn_abi_version": (_c_int, []),
    "gdn_last_error": (ctypes.c_char_p, []),
    "gdn_gates": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p,
                           _c_void_p, _c_int, _c_i64, _c_int, _c_void_p]),
    "gdn_frontend": (_c_int, [_c_void_p, _c_i64, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p,
                              _c_int, _c_i64, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int,
                              _c_int, _c_int, _c_int, _c_int, _c_void_p]),
    "gdn_scan_reference": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_void_p, _c_int, _c_void_p,
                                    _c_int, _c_void_p, _c_int, _c_void_p, _c_void_p, _c_int,
                                    _c_void_p, _c_int, _c_void_p, _c_int, _c_i64, _c_int, _c_int,
                                    _c_int, _c_int, _c_void_p]),
    "gdn_scan": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_void_p, _c_int, _c_void_p, _c_int,
                          _c_void_p, _c_int, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_int,
                          _c_void_p, _c_int, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_void_p]),
    "gdn_decode_step": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                 _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                 _c_void_p, _c_float, _c_void_p, _c_int, _c_int, _c_int, _c_int,
                                 _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_int, _c_void_p,
                                 _c_i64_p, _c_void_p, _c_void_p]),
    "gdn_pool_advance": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_int, _c_void_p]),
    "gdn_prefill_workspace_size": (_c_i64, [_c_int, _c_i64, _c_int, _c_int, _c_int, _c_int]),
    "gdn_prefill_chunked": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p,
                                     _c_int, _c_i64, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p,
                                     _c_void_p, _c_int, _c_void_p, _c_int, _c_i64, _c_int,
                                     _c_int, _c_int, _c_int, _c_void_p, _c_i64, _c_void_p]),
    "gdn_prefill_fused_workspace_size": (_c_i64, [_c_int, _c_i64, _c_int, _c_int, _c_int, _c_int]),
    "gdn_prefill_fused": (_c_int, [_c_void_p, _c_i64, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_int,
                                   _c_void_p, _c_void_p, _c_int, _c_i64, _c_void_p, _c_void_p,
                                   _c_void_p, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_int, _c_i64,
                                   _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_i64, _c_void_p]),
    "gdn_gated_rmsnorm": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_int, _c_i64, _c_int, _c_void_p, _c_float,
                                   _c_void_p, _c_int, _c_i64, _c_int, _c_void_p]),
    "gdn_quantized_matmul": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int,
                                      _c_void_p, _c_int, _c_void_p, _c_int, _c_int, _c_int, _c_int,
                                      _c_int, _c_void_p, _c_i64, _c_void_p]),
    "gdn_quantized_matmul_noalloc": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p,
                                              _c_int, _c_void_p, _c_int, _c_void_p, _c_int, _c_int,
                                              _c_int, _c_int, _c_int, _c_void_p]),
    "gdn_quantized_matmul_workspace_size": (_c_i64, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                                     _c_int]),
    "gdn_dequantize": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_int,
                                _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p]),
    "gdn_quantized_matmul_scheme": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int,
                                             _c_void_p, _c_int, _c_void_p, _c_int, _c_int, _c_int,
                                             _c_int, _c_int, _c_int, _c_void_p, _c_i64, _c_void_p]),
    "gdn_quantized_matmul_scheme_workspace_size": (_c_i64, [_c_int, _c_int, _c_int]),
}

EXPORTED = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib = None


class KernelError(RuntimeError):
    """A kernel entry point returned a non-zero status."""


def _hip_runtimes_mapped() -> set[str]:
    paths = set()
    with open("/proc/self/maps") as maps:
        for line in maps:
            if "libamdhip64.so" in line:
                paths.add(os.path.realpath(line.split()[-1]))
    return paths


def load(path: str = LIB_PATH):
    """Load and bind the library once per process (raises if it is absent)."""

    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise ImportError(
                f"{path} is missing: build the HIP kernels first "
                "(python mlx-lean-moe_amd/build.py, or __graft_entry__.build())")
        # The module-level `import torch` has mapped torch's libamdhip64; the
        # library's dependency resolves to it by SONAME, so both share one
        # HIP runtime (checked below).
        lib = ctypes.CDLL(path)
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if lib.gdn_abi_version() != ABI_VERSION:
            raise ImportError(f"{path}: ABI version {lib.gdn_abi_version()} != {ABI_VERSION}")
        runtimes = _hip_runtimes_mapped()
        if len(runtimes) > 1:
            raise ImportError(f"two HIP runtimes are mapped ({sorted(runtimes)}); "
                              "libgdn.so must share torch's")
        _lib = lib
        return lib


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float32, bfloat16 or float16") from None


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device):
    """The current stream of ``device`` as a raw pointer (torch's C accessor
    where it exists: the public ``current_stream`` builds a Stream object,
    ~5 us per call, several times per decode step)."""

    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


def call(name: str, *args) -> None:
    """Call an entry point and raise ``KernelError`` on a non-zero status."""

    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.gdn_last_error().decode(errors="replace")
        raise KernelError(f"{name} returned {rc}: {msg}")
