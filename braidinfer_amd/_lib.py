"""ctypes binding of the braidinfer_amd C ABI (include/braidinfer_amd.h).

This module is the only place that touches the shared library.  It loads
``braidinfer_amd/lib/libbraidinfer_amd.so`` (built by ``python -m
braidinfer_amd.build``), declares every entry point's argument types, and
turns a negative return code into a Python exception carrying
``bfa_last_error()``.  There is deliberately no CPU or PyTorch fallback: when
the library is missing, or a tensor is not on a ROCm device, the call raises.
"""
from __future__ import annotations

import ctypes
import threading
import warnings
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libbraidinfer_amd.so"
ABI_VERSION = 1

F32, F16, BF16, I32, I64 = 0, 1, 2, 3, 4
DTYPE_CODE = _DTYPE_CODE = {
    torch.float32: F32,
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.int32: I32,
    torch.int64: I64,
}
STATUS_INDEX_OOB = 1
STATUS_APPEND_SKIPPED = 2
LINEAR_PLAIN, LINEAR_SILU_AND_MUL = 0, 1
NOALLOC_SCRATCH_BYTES = 16 << 20  # BFA_NOALLOC_SCRATCH_BYTES

_P = c_void_p
# name -> (restype, argtypes); mirrors include/braidinfer_amd.h
_SIGNATURES = {
    "bfa_abi_version": (c_int, []),
    "bfa_last_error": (ctypes.c_char_p, []),
    "bfa_set_tuning": (c_int, [c_int, c_int]),
    "bfa_get_tuning": (c_int, [c_int]),
    "bfa_rms_norm": (c_int, [_P, _P, _P, c_int, c_int, c_int64, c_int64, c_int64,
                             c_int64, c_int64, c_int64, c_int64, c_float, _P]),
    "bfa_add_rms_norm": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int64, c_int64,
                                 c_int64, c_int64, c_int64, c_int64, c_float, _P]),
    "bfa_rms_norm_f32": (c_int, [_P, _P, _P, c_int, c_int, c_int64, c_int64, c_int64,
                                 c_int64, c_int64, c_int64, c_float, _P]),
    "bfa_embedding": (c_int, [_P, c_int64, c_int64, c_int64, c_int, _P, c_int, c_int64,
                              _P, c_int64, _P, _P]),
    "bfa_embedding_scaled": (c_int, [_P, c_int64, c_int64, c_int64, c_int, _P, c_int,
                                     c_int64, _P, c_int64, c_float, _P, _P]),
    "bfa_silu_and_mul": (c_int, [_P, _P, c_int, c_int64, c_int64, c_int64, c_int64, _P]),
    "bfa_rotary_embedding": (c_int, [_P, c_int, c_int64, _P, c_int64, c_int64, c_int,
                                     _P, c_int64, c_int64, c_int64, _P,
                                     _P, c_int64, c_int64, c_int64, _P, _P, _P]),
    "bfa_apply_rotary_emb": (c_int, [_P, c_int, c_int64, c_int64, c_int64, c_int64, c_int64,
                                     _P, _P, c_int64, _P, _P]),
    "bfa_rerotate_paged_k": (c_int, [_P, c_int, c_int64, c_int64, c_int64, c_int64,
                                     _P, c_int64, _P, _P, _P, c_int, c_int64,
                                     _P, c_int64, _P, c_int, c_float, _P, _P, _P]),
    "bfa_fused_rmsnorm_qkv_workspace_size": (c_int64, [c_int64, c_int64, c_int64, c_int64]),
    "bfa_fused_rmsnorm_qkv": (c_int, [_P, c_int, c_int64, c_int64, c_int64, _P, c_int,
                                      c_float, c_int, _P, c_int, c_int64, c_int64, _P, c_int,
                                      c_int64, c_int64, c_int, _P, _P, c_int, c_float, c_int,
                                      _P, c_int, _P, c_int64, _P, c_int, c_int64, _P,
                                      c_int64, _P, _P]),
    "bfa_fused_rmsnorm_qkv_noalloc": (c_int, [_P, c_int, c_int64, c_int64, c_int64, _P, c_int,
                                              c_float, c_int, _P, c_int, c_int64, c_int64, _P, c_int,
                                              c_int64, c_int64, c_int, _P, _P, c_int, c_float, c_int,
                                              _P, c_int, _P, c_int64, _P, c_int, c_int64, _P, _P]),
    "bfa_fold_rmsnorm_weight": (c_int, [_P, c_int, c_int64, c_int64, c_int64, _P, c_int, _P, c_int64, _P]),
    "bfa_rmsnorm_row_scale": (c_int, [_P, c_int, c_int64, c_int64, c_int64, _P, c_float, _P]),
    "bfa_fused_rmsnorm_qkv_folded": (c_int, [_P, c_int, c_int64, c_int64, c_int64, c_float, _P, c_int,
                                             c_int64, c_int64, _P, c_int, c_int64, c_int64, c_int,
                                             _P, c_int, _P, c_int64, _P, c_int, c_int64, _P, c_int64,
                                             _P, c_int, c_int64, c_int64, c_int64, c_int64, c_int64,
                                             c_int64, _P, c_int, c_int64, _P, _P, c_int, c_int64,
                                             _P, c_int, c_int64, c_int, _P, _P]),
    "bfa_rmsnorm_qkv_operand": (c_int, [_P, c_int, c_int64, c_int64, c_int64, _P, c_int,
                                        c_int, _P, c_int, c_float, _P]),
    "bfa_qkv_projection": (c_int, [_P, c_int64, c_int64, _P, c_int, c_int64, c_int64, _P,
                                   c_int, c_int64, c_int64, c_int, _P, _P, c_int, c_float,
                                   c_int, _P, c_int, _P, c_int64, _P, c_int, c_int64, _P,
                                   c_int64, _P, _P]),
    "bfa_append_paged_kv": (c_int, [_P, _P, c_int, c_int64, c_int64, c_int64, c_int64,
                                    c_int64, c_int64, c_int64, _P, c_int, c_int64, c_int64,
                                    c_int64, c_int64, c_int64, c_int64, _P, c_int, c_int64,
                                    _P, _P, c_int, c_int64,
                                    _P, c_int, c_int64, _P, _P]),
    "bfa_fused_rmsnorm_qkv_append_workspace_size": (c_int64, [c_int64, c_int64, c_int64, c_int64]),
    "bfa_fused_rmsnorm_qkv_append": (c_int, [_P, c_int, c_int64, c_int64, c_int64, _P, c_int,
                                             c_float, c_int, _P, c_int, c_int64, c_int64, _P, c_int,
                                             c_int64, c_int64, c_int, _P, _P, c_int, c_float, c_int,
                                             _P, c_int, _P, c_int64, _P, c_int, c_int64, _P, c_int64,
                                             _P, c_int, c_int64, c_int64, c_int64, c_int64, c_int64,
                                             c_int64, _P, c_int, c_int64, _P, _P, c_int, c_int64,
                                             _P, c_int, c_int64, c_int, _P, _P]),
    "bfa_online_softmax_update": (c_int, [_P, _P, _P, c_int, c_int, _P, _P, _P, _P, c_int, _P,
                                          c_int, c_int64, c_int64, c_int64, c_int64, c_int64,
                                          c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
                                          c_int64, c_int64, c_int64, c_int64, c_int64, c_float,
                                          c_int, _P]),
    "bfa_cascade_attention_workspace_size": (c_int64, [c_int64, c_int64, c_int64, c_int64,
                                                       c_int64, c_int64]),
    "bfa_cascade_attention": (c_int, [_P, c_int, c_int64, c_int64, c_int64, c_int64, _P, c_int,
                                      _P, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
                                      c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, c_int64,
                                      _P, c_int, c_float, c_float, c_int, _P, c_int64, _P,
                                      c_int64, _P, _P]),
    "bfa_linear_workspace_size": (c_int64, [c_int64, c_int64, c_int64, c_int]),
    "bfa_linear": (c_int, [_P, c_int, c_int64, c_int64, c_int64, _P, c_int64, c_int64, _P, c_int,
                           c_int, c_int, _P, c_int, c_int64, c_int, _P, c_int, c_int64, _P, c_int64,
                           _P]),
}

_lib = None
_lock = threading.Lock()


class BraidinferAMDError(RuntimeError):
    """A braidinfer_amd entry point returned an error code."""


def load():
    """Loads (once) and returns the ctypes handle of the C-ABI library."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"braidinfer_amd native library not found at {LIB_PATH}; "
                    "build it with `python -m braidinfer_amd.build` (hipcc, gfx950)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.bfa_abi_version() != ABI_VERSION:
                raise RuntimeError("braidinfer_amd: library ABI version mismatch; rebuild it")
            _lib = lib
    return _lib


def exported_symbols():
    """Names of every entry point this binding declares."""
    return list(_SIGNATURES)


def call(name: str, *args) -> int:
    """Calls entry point `name`; raises BraidinferAMDError on a negative return."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if name.endswith("workspace_size"):
        return rc
    if rc < 0:
        raise_error(rc)
    return rc


def entry(name: str):
    """The bound ctypes function of entry point `name`, for hot paths that call
    it directly and pass a negative return code to raise_error()."""
    return getattr(load(), name)


def raise_error(rc: int) -> None:
    msg = load().bfa_last_error().decode(errors="replace")
    if rc == -1:
        raise ValueError(msg)
    raise BraidinferAMDError(msg)


def workspace_size(name: str, *args) -> int:
    """`<name>(*args)` of a workspace-size entry point (not memoised: the plan
    it reflects also follows the planner overrides, see set_tuning)."""
    return getattr(load(), name)(*args)


# Planner overrides (BFA_TUNE_* of include/braidinfer_amd.h).  The library reads
# each from its environment variable (BFA_<NAME>) once, when it is loaded;
# set_tuning changes it afterwards.  For measurements and tests only.
TUNING_KEYS = {
    "DECODE_KS": 0, "DECODE_WG": 1, "DECODE_SPLITS": 2, "QKV_TILE": 3, "EDT_RT": 4,
    "DECODE_PAIR": 5, "NO_OPERAND_FOLD": 6, "CASCADE_DECODE_WG": 7, "CASCADE_FLAT": 8,
    "CASCADE_FLAT_WG": 9, "STREAM_STORES": 10, "QKV_PERSIST": 11,
    "DECODE_GEMV": 12,
}


_tuning_seen: dict = {}  # the values this module has read or set (the library changes them only through set_tuning)


def set_tuning(name: str, value: int | None) -> None:
    """Sets planner override `name` (a TUNING_KEYS key); None or -1 unsets it."""
    call("bfa_set_tuning", TUNING_KEYS[name], -1 if value is None else int(value))
    _tuning_seen.pop(name, None)


def get_tuning(name: str) -> int | None:
    """Current value of planner override `name`, None when unset (read from the
    library once, then remembered until set_tuning changes it)."""
    if name in _tuning_seen:
        return _tuning_seen[name]
    v = load().bfa_get_tuning(TUNING_KEYS[name])
    _tuning_seen[name] = None if v < 0 else v
    return _tuning_seen[name]


_workspaces: dict = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A device scratch buffer of at least `nbytes` (16-byte aligned) for a
    kernel launched on the current stream.  Outside graph capture one buffer
    per (device, stream) is kept and reused: launches on one stream are ordered,
    so a call's kernels finish with it before the next call's start.  Under
    graph capture a fresh allocation from the graph's pool is returned, so a
    captured graph never shares (or outlives) the eager buffer."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    stream = stream_of(device)
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)
    key = (idx, stream)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 16, 0 if buf is None else 2 * buf.numel()), dtype=torch.uint8,
                          device=device)
        _workspaces[key] = buf
    return buf


def clear_workspaces(device: torch.device | int | None = None) -> int:
    """Releases the reused scratch buffers of workspace() (all devices, or one)
    back to torch's caching allocator and returns the bytes released.  A buffer
    grows to the largest call made on its stream and is otherwise kept for the
    life of the process; call this after a one-off large call (an 8192-token
    cascade prefill, say) to give that memory back.  Safe while kernels that use
    a buffer are still queued: each buffer was allocated on the stream it serves,
    so the allocator reuses its memory only in that stream's order."""
    idx = None
    if device is not None:
        idx = device if isinstance(device, int) else (
            device.index if device.index is not None else torch.cuda.current_device())
    freed = 0
    for key in [k for k in _workspaces if idx is None or k[0] == idx]:
        freed += _workspaces.pop(key).numel()
    return freed


def dtype_code(t: torch.Tensor | torch.dtype) -> int:
    dt = t if isinstance(t, torch.dtype) else t.dtype
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"braidinfer_amd: unsupported dtype {dt}") from None


def ptr(t: torch.Tensor | None):
    """Device address of `t` (None for an absent optional tensor); ctypes turns
    the int into the void* the signature declares."""
    return None if t is None else t.data_ptr()


def require_device(*tensors: torch.Tensor | None) -> torch.device:
    """All given tensors must live on one ROCm device; returns it."""
    first = None
    idx = -1
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "braidinfer_amd ops run only on ROCm devices (got a tensor on "
                f"{t.device}); there is no CPU path")
        if first is None:
            first, idx = t, t.get_device()
        elif t.get_device() != idx:
            raise RuntimeError(f"braidinfer_amd: tensors on different devices ({first.device}, {t.device})")
    if first is None:
        raise RuntimeError("braidinfer_amd: no device tensor given")
    return first.device


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device):
    """Handle of the current torch stream on `device` (all work is enqueued there),
    read as the raw handle: building a torch Stream object for it took about 2 us
    per call, as much as the kernel launch itself."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


_status: dict[int, torch.Tensor] = {}


def status_word(device: torch.device) -> torch.Tensor:
    """The per-device int32 status word kernels OR error bits into."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    t = _status.get(idx)
    if t is None:
        t = torch.zeros(1, dtype=torch.int32, device=torch.device("cuda", idx))
        _status[idx] = t
    return t


def check_device_status(device: torch.device | int | None = None, reset: bool = True) -> None:
    """Synchronises with the device status word and raises IndexError if a
    kernel saw an out-of-range token id, position or delta since the last check."""
    if device is None:
        device = torch.device("cuda", torch.cuda.current_device())
    elif isinstance(device, int):
        device = torch.device("cuda", device)
    t = status_word(device)
    bits = int(t.item())
    if bits and reset:
        t.zero_()
    if bits & STATUS_APPEND_SKIPPED:
        # append_to_paged_kv_cache_custom prints an error for such a token and
        # carries on (kernels/kv_cache_utils.py:58-59); so does this check
        warnings.warn("braidinfer_amd: a KV append skipped a token whose page offset is "
                      "past the page list", RuntimeWarning, stacklevel=2)
    if bits & STATUS_INDEX_OOB:
        raise IndexError("braidinfer_amd: index out of range in a device kernel "
                         "(token id, rotary position, chunk delta or cache page)")
