"""ctypes binding of libnvs_amd.so (the C ABI declared in include/nvs_amd.h).

torch is imported first so that the library's libamdhip64.so.7 dependency resolves to the HIP runtime torch
already loaded: the streams and device pointers handed over below then belong to the same runtime.
"""
from __future__ import annotations

import ctypes
import pathlib
import threading

import torch  # noqa: F401  (loads the HIP runtime before the library)

from . import ABI_VERSION

LIB_PATH = pathlib.Path(__file__).resolve().with_name("libnvs_amd.so")

NVS_OK = 0
NVS_ERR_INVALID = -1
NVS_ERR_UNSUPPORTED = -2
NVS_ERR_WORKSPACE = -3
NVS_ERR_HIP = -4

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_size_p = ctypes.POINTER(ctypes.c_size_t)

# name -> argtypes, in the order of include/nvs_amd.h
SIGNATURES = {
    "nvs_abi_version": [],
    "nvs_last_error": [],
    "nvs_store_kvcache": [_p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i32, _i32, _i32, _p],
    "nvs_qk_norm_rope_store": [_p, _i64, _p, _i64, _p, _i64, _p, _p, _p, _f32, _p, _i64, _p, _p, _p, _i64, _i64, _i64,
                               _i64, _i64, _p, _i64, _p, _i64, _i64, _i32, _i32, _i32, _i32, _p],
    "nvs_paged_attention_workspace_size": [_i32, _i32, _i32, _i32, _i32, _i32, _size_p],
    "nvs_paged_attention": [_p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _i32, _p, _p, _p, _i32,
                            _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _p, _i64, _i64, _p, _p,
                            ctypes.c_size_t, _p],
    "nvs_probs_from_logits_workspace_size": [_i64, _i64, _i32, _size_p],
    "nvs_probs_from_logits": [_p, _i32, _i64, _i64, _i64, _i64, _p, _p, _p, _i32, _i32, _p, _p, ctypes.c_size_t, _p],
    "nvs_truncate_logits": [_p, _i64, _i64, _i64, _i64, _p, _p, _i32, _i32, _p, _p, ctypes.c_size_t, _p],
    "nvs_race": [_p, _i64, _p, _i64, _i64, _i64, _p, _p, _p, ctypes.c_size_t, _p],
    "nvs_race_workspace_size": [_i64, _i64, _size_p],
    "nvs_accept_random_workspace_size": [_i64, _i64, _size_p],
    "nvs_accept_random": [_p, _p, _p, _p, _p, _p, _i64, _i32, _i64, _i64, _p, _p, _p, _p, ctypes.c_size_t, _p],
    "nvs_accept_greedy_workspace_size": [_i64, _i64, _size_p],
    "nvs_accept_greedy": [_p, _i32, _i64, _p, _p, _i64, _i32, _i64, _i64, _p, _p, _p, ctypes.c_size_t, _p],
    "nvs_spec_accept_workspace_size": [_i64, _i32, _i64, _i64, _i32, _size_p],
    "nvs_spec_accept": [_p, _i32, _i64, _p, _p, _p, _i32, _i32, _p, _p, _p, _p, _p, _i64, _i32, _i64, _i64, _p, _p,
                        _p, _p, ctypes.c_size_t, _p],
    "nvs_spec_accept_candidates": [_p, _i32, _i64, _p, _p, _p, _i32, _i32, _p, _p, _i32, _i64, _p, _p, _p, _p, _i64,
                                   _i32, _i64, _i64, _p, _p, _p, _p, ctypes.c_size_t, _p],
    "nvs_spec_accept_noalloc": [_p, _i32, _i64, _p, _p, _p, _i32, _i32, _p, _p, _p, _p, _p, _i64, _i32, _i64, _i64,
                                _p, _p, _p],
    "nvs_markov_draw_workspace_size": [_i64, _i64, _i32, _size_p],
    "nvs_markov_draw": [_p, _i32, _i64, _p, _i64, _i64, _i64, _p, _p, _p, _i32, _i32, _i32, _p, _i64, _p, _p, _i64,
                        _p, _i64, _p, _p, ctypes.c_size_t, _p],
    "nvs_rms_norm": [_p, _i64, _p, _i64, _p, _f32, _p, _i64, _i64, _i32, _i32, _p],
    "nvs_silu_and_mul": [_p, _i64, _p, _i64, _i64, _i32, _i32, _p],
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class NvsError(RuntimeError):
    """A libnvs_amd call failed; .status is the nvs_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def load(path: pathlib.Path | str | None = None) -> ctypes.CDLL:
    """The loaded library (declared argument types, ABI version checked). Raises if it is not built."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        lib_path = pathlib.Path(path) if path is not None else LIB_PATH
        if not lib_path.exists():
            raise RuntimeError(f"{lib_path} is not built: run `python __graft_entry__.py build` (or "
                               "nano-vllm-speculative-decoding_amd/build.py) first")
        lib = ctypes.CDLL(str(lib_path))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        lib.nvs_last_error.restype = ctypes.c_char_p
        version = lib.nvs_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{lib_path} has ABI version {version}, expected {ABI_VERSION}: rebuild it")
        if path is None:
            _lib = lib
        return lib


def check(status: int, what: str) -> None:
    if status != NVS_OK:
        message = load().nvs_last_error().decode(errors="replace")
        raise NvsError(status, f"{what}: {message} (status {status})")


def size_out() -> ctypes.c_size_t:
    return ctypes.c_size_t(0)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return DTYPE_F32
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    if dtype == torch.float16:
        return DTYPE_F16
    raise ValueError(f"unsupported dtype {dtype}")


def require_device(*tensors: torch.Tensor | None) -> None:
    """The kernels only run on ROCm device tensors; a CPU tensor is an error, never a silent CPU path."""
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"nvs_amd kernels need ROCm device tensors, got a tensor on {t.device}")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


_persistent: dict = {}
# Buffers replaced by a larger one stay referenced until the process ends: a graph captured while one of them was
# current keeps its address in its kernel arguments, and every call leaves the buffer zero, so such a graph still
# replays correctly after a later, larger eager call grew the buffer.
_superseded: list = []


def persistent_workspace(name: str, nbytes: int, device: torch.device) -> torch.Tensor:
    """A zero-initialised device buffer kept across calls, for kernels that keep counters in it and leave them at
    zero when they finish (the row and unit counters of the one-launch accept, race and split-key attention). One
    buffer per (name, device); calls that share it must be ordered on one stream. It is created outside graph
    capture: warm up once eagerly before capturing. A buffer that is outgrown is replaced but never freed."""
    key = (name, device.type, device.index)
    buf = _persistent.get(key)
    if buf is None or buf.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"nvs_amd: the {name} workspace must be created before graph capture; "
                               "run the op once eagerly first")
        if buf is not None:
            _superseded.append(buf)
        buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        _persistent[key] = buf
    return buf
