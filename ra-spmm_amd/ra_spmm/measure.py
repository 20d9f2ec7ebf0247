"""Gather probe (measurement only; never on the routed path): how fast the
GPU gathers whole B rows in a given order with nothing else to do.  Over a
CSR's column indices it is the data-movement ceiling of any row-gathering
SpMM on that matrix.  Built from csrc/gather_probe.hip into
libra_gather_probe.so by build.py."""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = Path(__file__).resolve().parent / "libra_gather_probe.so"
        if not path.exists():
            raise ImportError(f"{path.name} is not built (python ra-spmm_amd/build.py)")
        lib = ctypes.CDLL(str(path))
        P = ctypes.c_void_p
        lib.ra_probe_out_elems.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32]
        lib.ra_probe_out_elems.restype = ctypes.c_int64
        lib.ra_probe_gather.argtypes = [P, ctypes.c_int64, ctypes.c_int32, P, ctypes.c_int64, ctypes.c_int32,
                                        P, P]
        lib.ra_probe_gather.restype = ctypes.c_int
        _LIB = lib
    return _LIB


class GatherProbe:
    """Gather rows idx[i] of B (fp32 [K, N], N in {16, 32, 64, 128, 256});
    each lane group walks `span` consecutive indices."""

    def __init__(self, B: torch.Tensor, idx: torch.Tensor, span: int = 32):
        K, N = B.shape
        if N % 4 or not 16 <= N <= 256 or (N // 4) & (N // 4 - 1):
            raise ValueError("the probe takes N in {16, 32, 64, 128, 256}")
        if B.dtype != torch.float32 or idx.dtype != torch.int32 or not (B.is_cuda and idx.is_cuda):
            raise ValueError("B fp32 and idx int32, both on the device")
        self.B, self.idx, self.packets, self.span = B.contiguous(), idx.contiguous(), N // 4, int(span)
        n = int(idx.numel())
        self.out = torch.empty(_lib().ra_probe_out_elems(n, self.packets, self.span) * 4, device=B.device)
        self.bytes = n * N * 4  # requested B bytes per call

    def run(self):
        st = _lib().ra_probe_gather(ctypes.c_void_p(self.B.data_ptr()), self.B.shape[1] // 4, self.packets,
                                    ctypes.c_void_p(self.idx.data_ptr()), self.idx.numel(), self.span,
                                    ctypes.c_void_p(self.out.data_ptr()),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if st != 0:
            raise RuntimeError("gather probe launch failed")
        return self.out
