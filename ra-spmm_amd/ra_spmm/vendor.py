"""rocSPARSE CSR SpMM as a comparator (measurement only; never on the routed
path).  The reference measures its speed-ups against the vendor library's
CSR SpMM (cuSPARSE CSR_ALG2, bindings/ra_bindings.cpp:431-615); on MI355X
that library is rocSPARSE.  Each algorithm rocSPARSE offers for CSR is timed
and the fastest is the comparator.  Built from csrc/vendor_spmm.cpp into
libra_vendor_spmm.so by build.py."""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

ALGS = {"default": 0, "csr": 1, "csr_row_split": 4, "csr_nnz_split": 5, "csr_merge_path": 9}
_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = Path(__file__).resolve().parent / "libra_vendor_spmm.so"
        if not path.exists():
            raise ImportError(f"{path.name} is not built (python ra-spmm_amd/build.py)")
        lib = ctypes.CDLL(str(path))
        P = ctypes.c_void_p
        I32, I64 = ctypes.c_int32, ctypes.c_int64
        lib.ra_vendor_spmm_create.argtypes = [P, P, P, P, P, I32, I32, I32, I64, I32, P, ctypes.POINTER(P)]
        lib.ra_vendor_spmm_create.restype = ctypes.c_int
        lib.ra_vendor_spmm_run.argtypes = [P, P]
        lib.ra_vendor_spmm_run.restype = ctypes.c_int
        lib.ra_vendor_spmm_set_dense.argtypes = [P, P, P]
        lib.ra_vendor_spmm_set_dense.restype = ctypes.c_int
        lib.ra_vendor_spmm_destroy.argtypes = [P]
        lib.ra_vendor_spmm_destroy.restype = None
        lib.ra_vendor_last_error.restype = ctypes.c_char_p
        _LIB = lib
    return _LIB


class RocsparseSpMM:
    """C = A @ B through rocsparse_spmm with one algorithm; the descriptors,
    buffer and preprocessing live as long as this object."""

    def __init__(self, rowptr, colind, vals, B, C, alg: str = "default"):
        for t, n in ((rowptr, "rowptr"), (colind, "colind")):
            if t.dtype != torch.int32 or not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{n} must be a contiguous int32 device tensor")
        for t, n in ((vals, "vals"), (B, "B"), (C, "C")):
            if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{n} must be a contiguous fp32 device tensor")
        self._keep = (rowptr, colind, vals, B, C)
        M, K, N = rowptr.numel() - 1, B.shape[0], B.shape[1]
        lib = _lib()
        h = ctypes.c_void_p()
        st = lib.ra_vendor_spmm_create(
            ctypes.c_void_p(rowptr.data_ptr()), ctypes.c_void_p(colind.data_ptr()),
            ctypes.c_void_p(vals.data_ptr()), ctypes.c_void_p(B.data_ptr()), ctypes.c_void_p(C.data_ptr()),
            M, K, N, colind.numel(), ALGS[alg], ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
            ctypes.byref(h))
        if st != 0:
            raise RuntimeError(f"rocsparse ({alg}): {lib.ra_vendor_last_error().decode()}")
        self._h = h

    def rebind(self, B, C):
        """Run on another B and C of the same shapes, dtype and device."""
        old = self._keep
        if B.shape != old[3].shape or C.shape != old[4].shape or B.dtype != torch.float32 \
                or C.dtype != torch.float32 or not (B.is_contiguous() and C.is_contiguous()):
            raise ValueError("rebind needs contiguous fp32 B and C of the plan's shapes")
        st = _lib().ra_vendor_spmm_set_dense(self._h, ctypes.c_void_p(B.data_ptr()), ctypes.c_void_p(C.data_ptr()))
        if st != 0:
            raise RuntimeError(f"rocsparse: {_lib().ra_vendor_last_error().decode()}")
        self._keep = old[:3] + (B, C)

    def run(self):
        # The current stream of this call, not the one current at creation.
        st = _lib().ra_vendor_spmm_run(self._h, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if st != 0:
            raise RuntimeError(f"rocsparse: {_lib().ra_vendor_last_error().decode()}")
        return self._keep[4]

    def close(self):
        if getattr(self, "_h", None):
            _lib().ra_vendor_spmm_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()


def fastest(rowptr, colind, vals, B, reps: int = 5):
    """The rocSPARSE algorithm that runs this A fastest at B's width, timed on
    B with HIP events: (plan bound to B and a fresh C, algorithm name)."""
    best = None
    for alg in ALGS:
        C = torch.empty((rowptr.numel() - 1, B.shape[1]), device=B.device)
        try:
            v = RocsparseSpMM(rowptr, colind, vals, B, C, alg)
        except RuntimeError:
            continue
        v.run()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            v.run()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        if best is None or ms < best[0]:
            if best is not None:
                best[1].close()
            best = (ms, v, alg)
        else:
            v.close()
    if best is None:
        raise RuntimeError("rocsparse: no CSR algorithm accepted this matrix")
    return best[1], best[2]
