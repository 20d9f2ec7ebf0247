"""The C-ABI library loads on a CPU-only host and exports every function the
public header declares; status/name helpers behave."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import torch  # noqa: F401  (share torch's HIP runtime, as in production)
from ra_spmm import capi

HEADER = Path(__file__).resolve().parents[1] / "include" / "ra_spmm.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ra_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_are_all_exported():
    lib = capi.load()
    names = declared_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(capi.EXPORTED) == names


def test_helpers():
    lib = capi.load()
    assert lib.ra_abi_version() == 1
    assert lib.ra_path_name(13) == b"ZERO_OVERHEAD_CSR"
    assert lib.ra_path_name(99) == b"UNKNOWN"
    assert lib.ra_reject_name(11) == b"NOT_IN_PORTFOLIO"
    assert lib.ra_status_string(4) == b"RA_ERR_UNSUPPORTED"


def test_invalid_arguments_return_status_not_crash():
    lib = capi.load()
    f = capi.Features()
    assert lib.ra_features_host(None, 5, 5, 5, ctypes.byref(f)) == 1
    assert b"rowptr" in lib.ra_last_error()
    rp = np.array([0, 2, 1], dtype=np.int32)  # non-monotone
    assert lib.ra_features_host(capi.ptr(rp), 2, 2, 2, ctypes.byref(f)) == 1
    info = capi.ZOInfo()
    assert lib.ra_zo_bins_host(capi.ptr(rp), 2, 2, None, None, None, None, ctypes.byref(info)) == 1
    h = ctypes.c_void_p()
    ci = np.array([0, 7, 1], dtype=np.int32)
    ok_rp = np.array([0, 2, 3], dtype=np.int32)
    vl = np.ones(3, dtype=np.float32)
    # Column index beyond K is rejected by the tile builder.
    assert lib.ra_tile_host_build(0, capi.ptr(ok_rp), capi.ptr(ci), capi.ptr(vl), 2, 4, 64, 1,
                                  ctypes.byref(h)) == 1
    r = capi.Route()
    assert lib.ra_route_dispatch(ctypes.byref(f), 0, 7, ctypes.byref(r)) == 1


def test_header_is_plain_c(tmp_path):
    """The boundary header compiles as ISO C99 on its own (no C++ and no HIP
    header in the signatures), so a C, cgo or FFI host can include it."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    src = tmp_path / "use_header.c"
    src.write_text('#include "ra_spmm.h"\nint main(void) { ra_tile_info i; ra_features f; (void)i; (void)f; '
                   'return ra_abi_version() == 1 ? 0 : 1; }\n')
    proc = subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", "-fsyntax-only",
                           "-I", str(HEADER.parent), str(src)],
                          capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
