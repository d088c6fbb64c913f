"""ctypes binding of libgdn_hip.so (the C ABI declared in include/gdn_hip.h).

The library is loaded from the package's ``lib/`` directory; it is built
in-tree by ``myvllm_amd.build.build()``.  ``MYVLLM_AMD_LIB`` in the environment
names another build of the same library instead (the host-AddressSanitizer
build of ``myvllm_amd.build.build_asan()``, for the C-ABI tests).  There is no
fallback: if the library is missing every op raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.environ.get("MYVLLM_AMD_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib",
                                                            "libgdn_hip.so")
ABI_VERSION = 1
MAX_NDIM = 4

# flags of gdn_chunk_prefill_ex (include/gdn_hip.h)
PREFILL_ZERO_INIT = 1
PREFILL_ACCUM_STATE = 2
PREFILL_ACCUM_OUT = 4

DTYPE_CODES = {
    torch.float32: 0,
    torch.bfloat16: 1,
    torch.float16: 2,
    torch.int32: 3,
    torch.int64: 4,
}

EXPORTED_SYMBOLS = (
    "gdn_recurrent_step",
    "gdn_chunk_prefill",
    "gdn_chunk_prefill_ex",
    "causal_conv1d_varlen",
    "causal_conv1d_step",
    "gdn_decode_step_fused",
    "causal_conv1d_varlen_qknorm",
    "gdn_rms_norm_gated",
    "gdn_gating",
    "flash_attention_varlen",
    "paged_attention_prefill",
    "paged_attention_decode_workspace_size",
    "paged_attention_decode",
    "paged_attention_decode_noalloc",
    "gdn_hbm_copy",
    "gdn_strerror",
    "gdn_abi_version",
)


class GdnTensor(ctypes.Structure):
    """Mirror of ``struct gdn_tensor``."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * MAX_NDIM),
        ("stride", ctypes.c_int64 * MAX_NDIM),
    ]


class GdnError(RuntimeError):
    """A non-zero return code of the C ABI (negative: validation, positive: HIP)."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with code {code}: {msg}")
        self.code = code


_lib = None
_lock = threading.Lock()
_PT = ctypes.POINTER(GdnTensor)


def load() -> ctypes.CDLL:
    """Load (once) and type the shared library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it first with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(or `python myvllm_amd/build.py`); there is no CPU fallback"
            )
        lib = ctypes.CDLL(LIB_PATH)
        lib.gdn_abi_version.restype = ctypes.c_int
        lib.gdn_abi_version.argtypes = []
        lib.gdn_strerror.restype = ctypes.c_char_p
        lib.gdn_strerror.argtypes = [ctypes.c_int]
        lib.gdn_recurrent_step.restype = ctypes.c_int
        lib.gdn_recurrent_step.argtypes = [_PT] * 8 + [ctypes.c_float, ctypes.c_void_p]
        lib.gdn_chunk_prefill.restype = ctypes.c_int
        lib.gdn_chunk_prefill.argtypes = [_PT] * 9 + [ctypes.c_float, ctypes.c_int32, ctypes.c_void_p]
        lib.gdn_chunk_prefill_ex.restype = ctypes.c_int
        lib.gdn_chunk_prefill_ex.argtypes = [_PT] * 9 + [ctypes.c_float] + [ctypes.c_int32] * 4 + [ctypes.c_void_p]
        lib.causal_conv1d_varlen.restype = ctypes.c_int
        lib.causal_conv1d_varlen.argtypes = [_PT] * 6 + [ctypes.c_void_p]
        lib.causal_conv1d_step.restype = ctypes.c_int
        lib.causal_conv1d_step.argtypes = [_PT] * 5 + [ctypes.c_void_p]
        lib.gdn_decode_step_fused.restype = ctypes.c_int
        lib.gdn_decode_step_fused.argtypes = [_PT] * 11 + [ctypes.c_int32, ctypes.c_float, ctypes.c_void_p]
        lib.causal_conv1d_varlen_qknorm.restype = ctypes.c_int
        lib.causal_conv1d_varlen_qknorm.argtypes = [_PT] * 6 + [ctypes.c_int64, ctypes.c_void_p]
        lib.gdn_rms_norm_gated.restype = ctypes.c_int
        lib.gdn_rms_norm_gated.argtypes = [_PT] * 4 + [ctypes.c_float, ctypes.c_void_p]
        lib.gdn_gating.restype = ctypes.c_int
        lib.gdn_gating.argtypes = [_PT] * 6 + [ctypes.c_void_p]
        lib.flash_attention_varlen.restype = ctypes.c_int
        lib.flash_attention_varlen.argtypes = [_PT] * 5 + [ctypes.c_int64, ctypes.c_float, ctypes.c_int32,
                                                           ctypes.c_void_p]
        lib.paged_attention_prefill.restype = ctypes.c_int
        lib.paged_attention_prefill.argtypes = [_PT] * 7 + [ctypes.c_int64, ctypes.c_float, ctypes.c_void_p]
        lib.paged_attention_decode_workspace_size.restype = ctypes.c_int64
        lib.paged_attention_decode_workspace_size.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                                              ctypes.c_int32]
        lib.paged_attention_decode.restype = ctypes.c_int
        lib.paged_attention_decode.argtypes = [_PT] * 7 + [ctypes.c_int32, ctypes.c_float, ctypes.c_void_p]
        lib.paged_attention_decode_noalloc.restype = ctypes.c_int
        lib.gdn_hbm_copy.restype = ctypes.c_int
        lib.gdn_hbm_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                     ctypes.c_void_p]
        lib.paged_attention_decode_noalloc.argtypes = [_PT] * 6 + [ctypes.c_int32, ctypes.c_float, ctypes.c_void_p]
        if lib.gdn_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {lib.gdn_abi_version()}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def strerror(code: int) -> str:
    return load().gdn_strerror(int(code)).decode()


def describe(t: torch.Tensor | None) -> GdnTensor:
    """Descriptor of a tensor (device pointer, dtype code, shape, element strides)."""
    d = GdnTensor()
    if t is None:
        return d
    if t.dim() > MAX_NDIM:
        raise ValueError(f"tensors of rank > {MAX_NDIM} are not supported")
    d.data = t.data_ptr() if t.numel() > 0 else None
    d.dtype = DTYPE_CODES.get(t.dtype, -1)
    d.ndim = t.dim()
    for i in range(t.dim()):
        d.shape[i] = t.shape[i]
        d.stride[i] = t.stride(i)
    return d


def check(fn: str, code: int) -> None:
    if code != 0:
        raise GdnError(fn, code, strerror(code))


def vec16(t: torch.Tensor) -> torch.Tensor:
    """t itself when the kernels can read it with 16-byte vector accesses (unit
    inner stride, 16-byte aligned data and outer strides), else a contiguous
    copy: the reference passes every stride to its kernels, so any strided
    input is accepted, at the cost of a copy when it is misaligned."""
    es = t.element_size()
    if t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((t.stride(i) * es) % 16 == 0 for i in range(t.dim() - 1)):
        return t
    return t.contiguous()


def vec16_ok(t: torch.Tensor) -> bool:
    return vec16(t) is t


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one HIP device (the kernels dereference the pointers)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("myvllm_amd ops take GPU tensors only (got a tensor on %s)" % t.device)
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
