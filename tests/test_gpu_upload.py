"""The plan builders' host-to-device upload (two pinned staging buffers, host
copy of one chunk overlapping the DMA of the other): the device tensor equals
torch's own copy for sizes below, at and across the 16 MiB chunks, and back to
back uploads (staging reuse) stay correct."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402


@pytest.mark.parametrize("n,dtype", [(1000, torch.int32), ((4 << 20) // 4 + 5, torch.int32), ((32 << 20) // 4, torch.float32),
                                     ((48 << 20) // 4 + 3, torch.int32), ((100 << 20) // 4 + 1, torch.float32)])
def test_upload_equals_torch_copy(n, dtype):
    rng = np.random.default_rng(n)
    src = torch.from_numpy(rng.integers(-(1 << 30), 1 << 30, n, dtype=np.int64).astype(np.int32))
    if dtype == torch.float32:
        src = src.view(torch.float32)
    outs = [ra_spmm._C.upload(src) for _ in range(3)]  # back to back: staging reuse
    torch.cuda.synchronize()
    ref = src.to("cuda")
    for out in outs:
        assert out.is_cuda and out.dtype == dtype and out.shape == src.shape
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32))
