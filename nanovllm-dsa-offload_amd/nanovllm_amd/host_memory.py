"""Pinned, device-mapped host memory for the DRAM KV caches.

The counterpart of ``torch_npu.empty_with_swapped_memory`` (reference
nanovllm/engine/model_runner.py:651-652, ut_ops/test_scatter_copy.py:64-72):
host DRAM that kernels dereference directly over the host link.

:func:`empty_host_mapped` returns a GPU-typed tensor over such memory, so it
passes the "same device" checks of the operators exactly like the
reference's swapped-memory tensors.  :func:`host_mapped_pair` additionally
returns a CPU tensor aliasing the same bytes, for filling the cache from the
host without a trip through the GPU.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


class _HostMappedBlock:
    """Owns one hipHostMalloc'd block; exposes it via __cuda_array_interface__."""

    def __init__(self, nbytes: int) -> None:
        host = ctypes.c_void_p()
        dev = ctypes.c_void_p()
        _lib.check(_lib.lib.nvdsa_host_mapped_alloc(nbytes, ctypes.byref(host), ctypes.byref(dev)))
        self.host = host.value
        self.dev = dev.value
        self.nbytes = nbytes
        self.__cuda_array_interface__ = {
            "shape": (nbytes // 2,),
            "typestr": "<i2",
            "data": (self.dev, False),
            "version": 3,
            "strides": None,
        }

    def __del__(self) -> None:
        if getattr(self, "host", None):
            _lib.lib.nvdsa_host_mapped_free(self.host)
            self.host = None


def _element_size(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()


def host_mapped_pair(shape, dtype: torch.dtype = torch.bfloat16, device=None):
    """Allocate host-mapped memory; return (gpu_tensor, cpu_alias).

    Both tensors alias the same pinned host bytes.  The GPU tensor is what
    the operators take; the CPU alias is for host-side initialisation.
    """
    if _element_size(dtype) != 2:
        raise ValueError("host-mapped KV caches hold 16-bit elements")
    shape = tuple(int(s) for s in shape)
    numel = 1
    for s in shape:
        numel *= s
    nbytes = max(numel * 2, 2)
    block = _HostMappedBlock(nbytes)
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    with torch.cuda.device(device):
        flat = torch.as_tensor(block, device=device)
    gpu = flat[:numel].view(dtype).view(shape)
    raw = (ctypes.c_uint8 * nbytes).from_address(block.host)
    cpu = torch.frombuffer(raw, dtype=torch.uint8)[: numel * 2].view(dtype).view(shape)
    # Keep the allocation alive as long as either view lives.
    cpu._nvdsa_block = block  # type: ignore[attr-defined]
    return gpu, cpu


def empty_host_mapped(shape, dtype: torch.dtype = torch.bfloat16, device=None) -> torch.Tensor:
    """GPU-typed tensor over pinned host memory (DRAM KV cache storage)."""
    gpu, _ = host_mapped_pair(shape, dtype, device)
    return gpu
