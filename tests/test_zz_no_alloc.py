"""ra_zo_plan_run_noalloc (the ZERO_OVERHEAD_CSR run that allocates nothing:
split-row partial slots in the library's fixed device array) against
ra_zo_plan_run, both through the C ABI.  Same kernels, so the results are
bit-identical; two calls in a row, the second on a smaller input, and the
over-limit case rejected before any launch."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402,F401  (loads torch's HIP runtime first)
from ra_spmm import capi  # noqa: E402
from ra_spmm import synthetic as S  # noqa: E402

P = capi.ptr


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _run_both(lib, g, N, seed):
    rp, ci, vl = g.torch("cuda")
    plan = ctypes.c_void_p()
    capi.check(lib.ra_zo_plan_create_device(P(rp), g.M, g.K, _stream(), ctypes.byref(plan)))
    info = capi.ZOInfo()
    capi.check(lib.ra_zo_plan_get_info(plan, ctypes.byref(info)))
    B = torch.from_numpy(np.random.default_rng(seed).standard_normal((g.K, N)).astype(np.float32)).cuda()
    ref = torch.empty(g.M, N, device="cuda")
    got = torch.full((g.M, N), float("nan"), device="cuda")
    capi.check(lib.ra_zo_plan_run(plan, P(rp), P(ci), P(vl), P(B), P(ref), N, _stream()))
    capi.check(lib.ra_zo_plan_run_noalloc(plan, P(rp), P(ci), P(vl), P(B), P(got), N, _stream()))
    torch.cuda.synchronize()
    lib.ra_zo_plan_destroy(plan)
    return info, ref.cpu().numpy(), got.cpu().numpy()


def test_noalloc_equals_allocating_run_twice():
    lib = capi.load()
    big = S.random_csr(6000, 5000, 20.0, seed=41, skew=0.8, empty_frac=0.02, max_deg=3000)
    small = S.random_csr(900, 1200, 14.0, seed=42, skew=0.9, max_deg=1100)
    for g, N, seed in ((big, 256, 1), (small, 64, 2), (small, 47, 3)):
        print(f"[noalloc] M={g.M} N={N}", flush=True)
        info, ref, got = _run_both(lib, g, N, seed)
        assert info.num_split_chunks > 0  # the fixed array is in use
        np.testing.assert_array_equal(got, ref)


def test_noalloc_rejects_more_than_its_scratch():
    lib = capi.load()
    deg = np.full(2000, 300, np.int64)  # 2000 split rows of 2 chunks each
    rowptr = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    colind = np.tile(np.arange(300, dtype=np.int32), 2000)
    rp = torch.from_numpy(rowptr).cuda()
    ci = torch.from_numpy(colind).cuda()
    vl = torch.ones(colind.size, device="cuda")
    plan = ctypes.c_void_p()
    capi.check(lib.ra_zo_plan_create_device(P(rp), 2000, 300, _stream(), ctypes.byref(plan)))
    info = capi.ZOInfo()
    capi.check(lib.ra_zo_plan_get_info(plan, ctypes.byref(info)))
    N = 4200  # 4000 slots x 4200 x 4 bytes > 64 MiB
    assert info.num_split_chunks * N * 4 > 64 << 20
    one = torch.zeros(1, device="cuda")
    st = lib.ra_zo_plan_run_noalloc(plan, P(rp), P(ci), P(vl), P(one), P(one), N, _stream())
    assert st == 4  # RA_ERR_UNSUPPORTED
    assert b"64 MiB" in lib.ra_last_error()
    lib.ra_zo_plan_destroy(plan)
