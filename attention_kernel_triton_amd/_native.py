"""ctypes binding of libakt_amd.so (the C ABI declared in include/akt_amd.h).

The library is loaded after torch, so it binds to the HIP runtime torch has
already loaded (both carry the soname libamdhip64.so.7).  There is no fallback
path: if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libakt_amd.so"

AKT_OK = 0
_ERRORS = {1: "invalid argument", 2: "unsupported", 3: "workspace", 4: "HIP error"}

_i64 = C.c_int64
_p = C.c_void_p
_i64x = C.POINTER(C.c_int64)

# name -> (restype, argtypes)
_SIGNATURES = {
    "akt_last_error": (C.c_char_p, []),
    "akt_abi_version": (C.c_int, []),
    "akt_prefill_fwd": (C.c_int, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                  _i64x, _i64x, _i64x, _i64x, C.c_float, C.c_int, _p, C.c_int, _p]),
    "akt_prefill_fwd_lse": (C.c_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                      _i64x, _i64x, _i64x, _i64x, _i64x, C.c_float, C.c_int, _p,
                                      C.c_int, _p]),
    "akt_prefill_fwd_ex": (C.c_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                     _i64x, _i64x, _i64x, _i64x, _i64x, C.c_float, C.c_int, _p,
                                     C.c_int, C.c_int, _p]),
    "akt_merge_states": (C.c_int, [_p, C.c_int, _p, _p, C.c_int, _p, _i64, _i64, _i64, _i64x,
                                   _i64x, _i64, _i64, _p]),
    "akt_decode_workspace_size": (C.c_size_t, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "akt_decode_fwd": (C.c_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                 _i64x, _i64x, _i64x, C.c_float, _i64, _p, C.c_size_t, _p]),
    "akt_decode_paged_workspace_size": (C.c_size_t, [_i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "akt_decode_paged_fwd": (C.c_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                       _i64, _i64, _i64x, _i64x, C.c_float, _i64, _p, C.c_size_t, _p]),
    "akt_decode_paged_fwd_noalloc": (C.c_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64,
                                               _i64, _i64, _i64, _i64x, _i64x, C.c_float, _i64,
                                               _p]),
    "akt_sparse_decode_workspace_size": (C.c_size_t, [_i64, _i64, _i64, _i64, _i64]),
    "akt_sparse_decode_fwd": (C.c_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                        _i64, _i64x, _i64x, _i64x, _i64x, _i64x, C.c_float, _i64,
                                        _p, C.c_size_t, _p]),
    "akt_sparse_decode_paged_fwd": (C.c_int, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64,
                                              _i64, _i64, _i64, _i64, _i64x, _i64x, _i64x, _i64x,
                                              C.c_float, _i64, _p, C.c_size_t, _p]),
    "akt_magicpig_decode_paged_fwd": (C.c_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64,
                                                _i64, _i64, _i64, _i64, _i64, _i64, _i64x, _i64x,
                                                _i64x, _i64x, _i64, _p, C.c_size_t, _p]),
    "akt_sparse_decode_csr_fwd": (C.c_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64,
                                            _i64, _i64, _i64x, _i64x, _i64x, C.c_float, _i64, _p,
                                            C.c_size_t, _p]),
    "akt_sparse_decode_paged_csr_fwd": (C.c_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64,
                                                  _i64, _i64, _i64, _i64, _i64, _i64, _i64x,
                                                  _i64x, _i64, _p, C.c_size_t, _p]),
    "akt_paged_kv_append": (C.c_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                      _i64, _i64x, _i64x, _i64x, _p]),
    "akt_kept_index_from_mask": (C.c_int, [_p, _i64, _i64, _i64, _p, _p, _i64, _p, C.c_int, _p]),
    "akt_kept_index_from_uniform": (C.c_int, [_p, C.c_float, _i64, _i64, _i64, _p, _p, _i64, _p,
                                              C.c_int, _p]),
    "akt_diag_paged_gather": (C.c_int, [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64x, _p, _p]),
    "akt_diag_stream_read": (C.c_int, [_p, _i64, _p, _p]),
    "akt_kernel_timer_enable": (C.c_int, [C.c_int]),
    "akt_kernel_timer_read": (C.c_int, [C.POINTER(C.c_double), C.POINTER(C.c_int64)]),
}

_lib = None


# Version of include/akt_amd.h these bindings follow (AKT_ABI_VERSION).
ABI_VERSION = 2
# Bytes at the start of a decode workspace that must be zero before its first
# use (AKT_WORKSPACE_ZERO_BYTES: the counter header and the arrival counters).
WORKSPACE_ZERO_BYTES = 256 + 32768 * 4


def library_path() -> Path:
    return LIB_PATH


def load() -> C.CDLL:
    """Load libakt_amd.so once and attach the C signatures."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"{path} is not built: run `python -m attention_kernel_triton_amd.build` "
            "(the HIP kernels have no fallback implementation)")
    # Global symbols: the compiled host layer (_akt_torch) resolves its akt_*
    # calls against this library.
    lib = C.CDLL(str(path), mode=C.RTLD_GLOBAL)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.akt_abi_version() != ABI_VERSION:
        raise RuntimeError(
            f"{path} has ABI version {lib.akt_abi_version()}, these bindings need "
            f"{ABI_VERSION}: rebuild with `python -m attention_kernel_triton_amd.build`")
    _lib = lib
    return lib


_ext = None


def torch_ext():
    """The compiled host layer of the hot entry points (module ``_akt_torch``,
    built from csrc/torch_ops.cpp), loaded after libakt_amd.so."""
    global _ext
    if _ext is None:
        load()
        try:
            from . import _akt_torch
        except ImportError as e:
            raise RuntimeError(
                "the host layer _akt_torch is not built: run "
                "`python -m attention_kernel_triton_amd.build`") from e
        _ext = _akt_torch
    return _ext


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(rc: int, what: str) -> None:
    if rc != AKT_OK:
        msg = load().akt_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({_ERRORS.get(rc, rc)}): {msg}")


def strides(t: torch.Tensor, n: int | None = None):
    s = list(t.stride())
    if n is not None:
        s = s[:n]
    return (C.c_int64 * len(s))(*s)


def i64s(*vals):
    return (C.c_int64 * len(vals))(*vals)


def ptr(t: torch.Tensor | None):
    return None if t is None else C.c_void_p(t.data_ptr())


# torch's raw current-stream query (what Triton's launcher uses) skips building
# a Stream object: ~0.2 us instead of ~1.8 us per call.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor):
    """The current HIP stream of ``t``'s device, as a ctypes pointer."""
    idx = t.device.index
    if idx is None:
        idx = torch.cuda.current_device()
    if _raw_stream is not None:
        return C.c_void_p(_raw_stream(idx))
    return C.c_void_p(torch.cuda.current_stream(idx).cuda_stream)


_WS_CACHE: dict = {}


def workspace(nbytes: int, device, stream=None) -> torch.Tensor | None:
    """Decode workspace for ``stream`` (default: the current stream of ``device``).

    The C ABI requires the workspace's first WORKSPACE_ZERO_BYTES (its
    counters) to be zero before first use (each call leaves them zero) and a
    workspace to be reused only by calls ordered on one stream, so one
    zero-initialised buffer is kept per (device, stream) and grown when a call
    needs more.  ``stream`` is
    the value ``stream_of`` returned for the same call.
    """
    if nbytes == 0:
        return None
    dev = torch.device(device)
    if dev.index is None:
        dev = torch.device(dev.type, torch.cuda.current_device())
    if stream is None:
        stream = C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    key = (dev.index, stream.value)
    buf = _WS_CACHE.get(key)
    if buf is None or buf.numel() < nbytes:
        size = max(int(nbytes), 2 * buf.numel() if buf is not None else 0)
        buf = torch.zeros(size, dtype=torch.uint8, device=dev)
        _WS_CACHE[key] = buf
    return buf


def workspace_buffers():
    """(device index, stream handle, buffer) of every cached decode workspace:
    those of the Python wrappers (``workspace``) and of the compiled host layer."""
    out = [(k[0], k[1] or 0, v) for k, v in _WS_CACHE.items()]
    if _ext is not None:
        out += [(d, s, b) for d, s, b in _ext.workspaces()]
    return out


class kernel_timer:
    """Context manager: HIP-event time of each entry point's dominant kernel.

    >>> with kernel_timer() as t:
    ...     run()
    >>> t.total_ms, t.launches
    """

    def __enter__(self):
        check(load().akt_kernel_timer_enable(1), "akt_kernel_timer_enable")
        self.total_ms, self.launches = 0.0, 0
        return self

    def __exit__(self, *exc):
        lib = load()
        ms, n = C.c_double(0.0), C.c_int64(0)
        rc = lib.akt_kernel_timer_read(C.byref(ms), C.byref(n))
        lib.akt_kernel_timer_enable(0)
        check(rc, "akt_kernel_timer_read")
        self.total_ms, self.launches = ms.value, n.value
        return False
