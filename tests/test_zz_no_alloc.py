"""fim_calibrate_block32_noalloc (the allocation-free variant of fim_calibrate_block32, its amax words in a file-scope
device scratch array) called through the C ABI: on two calls in a row, the second with a smaller input, its exponents
equal those of the workspace entry point byte for byte, and those equal the oracle's (quant/formats/mx.py:41-47)."""

import pytest
import torch

from flashim_amd import _lib
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _both(x: torch.Tensor):
    lib = _lib.load()
    rows, c = x.shape
    groups = -(-c // 32)
    stream = torch.cuda.current_stream().cuda_stream
    want = torch.full((groups,), 99, dtype=torch.int8, device=DEV)
    workspace = torch.empty(groups, dtype=torch.int32, device=DEV)
    code = _lib.DTYPE_CODES[x.dtype]
    assert lib.fim_calibrate_block32(x.data_ptr(), code, rows, c, x.stride(0), workspace.data_ptr(), want.data_ptr(),
                                     stream) == 0
    got = torch.full((groups,), 99, dtype=torch.int8, device=DEV)
    assert lib.fim_calibrate_block32_noalloc(x.data_ptr(), code, rows, c, x.stride(0), got.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    return got.cpu(), want.cpu()


def test_noalloc_calibration_matches_workspace_entry_point_twice():
    torch.manual_seed(0)
    big = (torch.randn(20000, 4096) * torch.rand(4096) * 50).to(torch.bfloat16)  # 128 groups, the larger call first
    small = (torch.randn(300, 96) * 0.01).float()  # far smaller amax: stale words from the first call would show
    for x in (big, small):
        got, want = _both(x.to(DEV))
        assert torch.equal(got, want)
        assert torch.equal(got, ref.calibrate_block32_exponent(x))


def test_noalloc_calibration_at_its_size_limit_and_past_it():
    lib = _lib.load()
    torch.manual_seed(1)
    x = torch.randn(4, 131072, device=DEV)
    got, want = _both(x)
    assert torch.equal(got, want)
    out = torch.empty(4097, dtype=torch.int8, device=DEV)
    wide = torch.empty(1, 131073, device=DEV)
    assert lib.fim_calibrate_block32_noalloc(wide.data_ptr(), 0, 1, 131073, 131073, out.data_ptr(),
                                             torch.cuda.current_stream().cuda_stream) == _lib.FIM_ERR_UNSUPPORTED
