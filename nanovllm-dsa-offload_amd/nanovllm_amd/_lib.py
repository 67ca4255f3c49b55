"""ctypes binding of libnvdsa.so (the C ABI declared in include/nvdsa.h).

Loading order matters: torch is imported first so that the HIP runtime torch
ships with (SONAME libamdhip64.so.7) is already resident and libnvdsa.so binds
to that same runtime instead of loading a second copy.

There is no fallback: if the library is missing this module raises, and every
operator that needs it fails loudly.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  -- must precede the CDLL load (shared HIP runtime)

LIB_PATH = Path(__file__).resolve().parent / "libnvdsa.so"

# nvdsa_dtype
INT32, FLOAT16, BFLOAT16, FLOAT32 = 0, 1, 2, 3
HOST_MAPPED_DEVICE = -1
_NOT_DEVICE = -2  # ordinary (pageable) CPU memory: rejected by every entry point

STATUS_NAMES = {
    0: "OK",
    1: "SHAPE",
    2: "DTYPE",
    3: "LAYOUT",
    4: "DEVICE",
    5: "WORKSPACE",
    6: "RUNTIME",
    7: "ARG",
}


class NvdsaTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 4),
        ("contiguous", ctypes.c_int32),
        ("device", ctypes.c_int32),
    ]


_P = ctypes.POINTER(NvdsaTensor)
_VP = ctypes.c_void_p
_SZ = ctypes.c_size_t
_I64 = ctypes.c_int64
_DBL = ctypes.c_double

# (name, argtypes) of every exported entry point; restype is int unless noted.
SIGNATURES = {
    "nvdsa_last_error": ([], ctypes.c_char_p),
    "nvdsa_version": ([], ctypes.c_char_p),
    "nvdsa_fused_li_manage_workspace_size": ([_I64, _I64, _I64], _SZ),
    "nvdsa_fused_li_manage": ([_P] * 11 + [_VP, _SZ, _VP], ctypes.c_int),
    "nvdsa_fused_li_manage_noalloc": ([_P] * 11 + [_VP], ctypes.c_int),
    "nvdsa_fused_li_manage_mtp_workspace_size": ([_I64, _I64, _I64], _SZ),
    "nvdsa_fused_li_manage_mtp": ([_P] * 13 + [_VP, _SZ, _VP], ctypes.c_int),
    "nvdsa_scatter_copy": ([_P] * 9 + [_VP], ctypes.c_int),
    "nvdsa_sparse_tail_attention_workspace_size": ([_I64, _I64, _I64], _SZ),
    "nvdsa_sparse_tail_attention": ([_P] * 9 + [_DBL, _P, _VP, _SZ, _VP], ctypes.c_int),
    "nvdsa_sparse_tail_attention_mtp": ([_P] * 9 + [_DBL, _P, _VP, _SZ, _VP], ctypes.c_int),
    "nvdsa_fused_copy_sfa": ([_P] * 14 + [_DBL, _P, _VP, _SZ, _VP], ctypes.c_int),
    "nvdsa_fused_copy_sfa_mtp": ([_P] * 16 + [_DBL, _P, _VP, _SZ, _VP], ctypes.c_int),
    "nvdsa_initialize_lidu_row_workspace_size": ([_I64], _SZ),
    "nvdsa_initialize_lidu_row": ([_P] * 4 + [_I64, _I64] + [_P] * 7 + [_I64, _VP, _SZ, _VP], ctypes.c_int),
    "nvdsa_initialize_lidu_row_shared": ([_P, _I64] + [_P] * 6 + [_VP, _SZ, _VP], ctypes.c_int),
    "nvdsa_dsa_indexer_query_rope_inplace": ([_P] * 3 + [_I64, _VP], ctypes.c_int),
    "nvdsa_dsa_indexer_project_query_only": ([_P] * 8 + [_I64, _I64, _I64, _DBL, _VP], ctypes.c_int),
    "nvdsa_persist_prefill_blocks": ([_P] * 6 + [_VP], ctypes.c_int),
    "nvdsa_host_mapped_alloc": ([_SZ, ctypes.POINTER(_VP), ctypes.POINTER(_VP)], ctypes.c_int),
    "nvdsa_host_mapped_free": ([_VP], ctypes.c_int),
    "nvdsa_profile_begin": ([ctypes.c_int32], ctypes.c_int),
    "nvdsa_profile_end": ([ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int32), ctypes.c_int32,
                           ctypes.POINTER(ctypes.c_int32)], ctypes.c_int),
    "nvdsa_kernel_name": ([ctypes.c_int32], ctypes.c_char_p),
    "nvdsa_xcd_roles": ([ctypes.POINTER(ctypes.c_uint32), ctypes.c_int32], ctypes.c_int),
    "nvdsa_xcd_roles_record": ([ctypes.c_int32], None),
}


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is not built. Run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(or nanovllm-dsa-offload_amd/csrc/build.py) first."
        )
    lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    return lib


lib = _load()

_DTYPE_CODES = {
    torch.int32: INT32,
    torch.float16: FLOAT16,
    torch.bfloat16: BFLOAT16,
    torch.float32: FLOAT32,
}


def describe(t: torch.Tensor) -> NvdsaTensor:
    """Plain-C descriptor of a torch tensor (device pointer, dtype, shape)."""
    d = NvdsaTensor()
    d.data = t.data_ptr() if t.numel() else (t.data_ptr() or None)
    d.dtype = _DTYPE_CODES.get(t.dtype, -1)
    nd = t.dim()
    d.ndim = nd if nd <= 4 else 5
    for i in range(min(nd, 4)):
        d.shape[i] = t.shape[i]
    d.contiguous = 1 if t.is_contiguous() else 0
    if t.is_cuda:
        d.device = t.device.index if t.device.index is not None else torch.cuda.current_device()
    elif t.device.type == "cpu" and _is_pinned(t):
        d.device = HOST_MAPPED_DEVICE
    else:
        d.device = _NOT_DEVICE
    return d


def _is_pinned(t: torch.Tensor) -> bool:
    try:
        return bool(t.is_pinned())
    except RuntimeError:
        return False


def last_error() -> str:
    msg = lib.nvdsa_last_error()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    """Raise like a failing TORCH_CHECK when an entry point reports an error."""
    if status != 0:
        raise RuntimeError(f"[nvdsa {STATUS_NAMES.get(status, status)}] {last_error()}")


def version() -> str:
    return lib.nvdsa_version().decode()


class KernelTimer:
    """Per-kernel HIP event timing of the entry points called inside a
    ``with`` block on this thread (nvdsa_profile_begin / nvdsa_profile_end)."""

    def __init__(self, capacity: int = 4096) -> None:
        self.capacity = capacity
        self.records: list[tuple[str, float]] = []

    def __enter__(self) -> "KernelTimer":
        check(lib.nvdsa_profile_begin(self.capacity))
        return self

    def __exit__(self, *exc) -> None:
        ms = (ctypes.c_float * self.capacity)()
        ids = (ctypes.c_int32 * self.capacity)()
        n = ctypes.c_int32()
        check(lib.nvdsa_profile_end(ms, ids, self.capacity, ctypes.byref(n)))
        self.records = [(lib.nvdsa_kernel_name(ids[i]).decode(), float(ms[i])) for i in range(n.value)]

    def mean_ms(self, name: str) -> float:
        vals = [ms for k, ms in self.records if k == name]
        return sum(vals) / len(vals) if vals else float("nan")


class record_xcd_roles:
    """Context manager: the MTP3 overlap kernels launched inside the block
    record the XCDs their workgroup roles ran on (nvdsa_xcd_roles_record);
    recording is off again afterwards.  Read the record with xcd_roles."""

    def __enter__(self):
        lib.nvdsa_xcd_roles_record(1)
        return self

    def __exit__(self, *exc) -> None:
        lib.nvdsa_xcd_roles_record(0)


def xcd_roles(reset: bool = False) -> tuple[int, int]:
    """(copy, attention) bit masks of the XCDs the MTP3 overlap kernel's two
    workgroup roles ran on, on the current device, since the last reset
    (nvdsa_xcd_roles).  Disjoint masks mean the dispatcher dealt workgroups to
    the XCDs round-robin, as the kernel's role split assumes.  Synchronises
    the device."""
    masks = (ctypes.c_uint32 * 2)()
    check(lib.nvdsa_xcd_roles(masks, int(reset)))
    return int(masks[0]), int(masks[1])


def exported_symbols_from_header(header: os.PathLike | str) -> list[str]:
    """Names of the functions declared in include/nvdsa.h."""
    import re

    text = Path(header).read_text()
    return sorted(set(re.findall(r"\b(nvdsa_[a-z0-9_]+)\s*\(", text)))
