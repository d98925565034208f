"""Device numerics: the hardware E4M3 conversion the kernels use agrees byte for byte with the software encoder and
with torch (every BF16 value and random FP32 values, subnormals and signed zeros included), and the device MX
exponent rule agrees with the oracle's ceil(log2(amax / 448)) at every power-of-two boundary."""

import pytest
import torch

from flashim_amd import _lib
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _device_e4m3(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    x = x.to(DEV).float().contiguous()
    out = torch.empty(2 * x.numel(), device=DEV, dtype=torch.uint8)
    _lib.probe_call("fim_test_e4m3", x.data_ptr(), x.numel(), out.data_ptr(), _lib.stream_of(x))
    out = out.cpu()
    return out[: x.numel()], out[x.numel():]


def test_e4m3_hardware_matches_software_and_torch():
    bf16 = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    bf16 = bf16[torch.isfinite(bf16)].clamp(-448, 448)
    torch.manual_seed(0)
    rnd = (torch.randn(1 << 21) * torch.exp2(torch.randint(-24, 10, (1 << 21,)).float())).clamp(-448, 448)
    ties = torch.tensor([2.0**-10, -(2.0**-10), 3 * 2.0**-10, 0.0, -0.0, 448.0, -448.0, 1.0625, 1.1875, 2.0**-6])
    for x in (bf16, rnd, ties):
        hw, sw = _device_e4m3(x)
        want = x.to(torch.float8_e4m3fn).view(torch.uint8)
        assert torch.equal(sw, want)
        assert torch.equal(hw, want), f"{(hw != want).sum().item()} hardware E4M3 mismatches"


def test_mx_exponent_matches_oracle():
    torch.manual_seed(0)
    ks = torch.arange(-149, 128).double()
    bnd = (torch.exp2(ks)[:, None] * (1 + torch.arange(0, 64).double()[None] * 2.0**-23) * 448).float().flatten()
    amax = torch.cat([
        torch.tensor([0.0, 448.0, 449.0, 1.0, 1e-30, 1e-45, 3e38]),
        torch.rand(1 << 20) * torch.exp2(torch.randint(-140, 120, (1 << 20,)).float()),
        bnd, bnd.nextafter(torch.tensor(0.0)), bnd.nextafter(torch.tensor(3e38)),
    ])
    amax = amax[torch.isfinite(amax)].contiguous()
    out = torch.empty(amax.numel(), device=DEV, dtype=torch.int8)
    a = amax.to(DEV)
    _lib.probe_call("fim_test_mx_exponent", a.data_ptr(), a.numel(), out.data_ptr(), _lib.stream_of(a))
    assert torch.equal(out.cpu(), ref.scale_exponent_from_amax(amax))


def test_bf16_hardware_rounding_matches_torch():
    """v_cvt_pk_bf16_f32 (the epilogues' rounding) vs the software rule and torch: every BF16 value and its midpoints
    to the neighbours (the tie cases), their one-ulp perturbations, FP32 subnormals and random values."""
    base = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    base = base[torch.isfinite(base)]
    bits = base.view(torch.int32)
    mids = (bits + 0x8000).view(torch.float32)
    cases = [base, mids, (bits + 0x7FFF).view(torch.float32), (bits + 0x8001).view(torch.float32),
             torch.randint(1, 1 << 23, (1 << 16,), dtype=torch.int32).view(torch.float32),
             torch.randn(1 << 20) * torch.exp2(torch.randint(-140, 120, (1 << 20,)).float())]
    for x in cases:
        x = x[torch.isfinite(x)].contiguous()
        xd = x.to(DEV)
        out = torch.empty(2 * x.numel(), device=DEV, dtype=torch.int16)
        _lib.probe_call("fim_test_bf16", xd.data_ptr(), x.numel(), out.data_ptr(), _lib.stream_of(xd))
        out = out.cpu()
        want = x.to(torch.bfloat16).view(torch.int16)
        assert torch.equal(out[x.numel():], want)
        assert torch.equal(out[: x.numel()], want), f"{(out[: x.numel()] != want).sum().item()} hardware BF16 mismatches"


def test_gelu_within_one_bf16_rounding_of_torch_on_every_bf16_input():
    """The epilogues' GELU vs F.gelu on a BF16 tensor over all finite BF16 inputs: within one BF16 rounding of
    torch's value or an absolute 2^-12 (torch's negative tail, where 1 + erf cancels)."""
    x = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16)
    xd = x.to(DEV)
    out = torch.empty(65536, device=DEV, dtype=torch.int16)
    _lib.probe_call("fim_test_gelu", xd.data_ptr(), 65536, out.data_ptr(), _lib.stream_of(xd))
    xs = x.view(torch.bfloat16)
    want = torch.nn.functional.gelu(xs).float()
    got = out.cpu().view(torch.bfloat16).float()
    ok = torch.isfinite(xs.float()) & (xs.float().abs() < 1e30)
    diff = (got - want).abs()[ok]
    assert (diff <= want.abs()[ok] * 2**-7 + 2**-12).all()
    assert (got[ok] != want[ok]).float().mean() < 0.02


@pytest.mark.gpu
@pytest.mark.parametrize("kind", [0, 1, 2])
def test_mfma_peak_hook_runs(kind):
    """The MFMA microbenchmark the bench quotes its measured peaks from: it runs and every thread's sum is finite."""
    out = torch.empty(4 * 256, device="cuda", dtype=torch.float32)
    _lib.probe_call("fim_test_mfma_peak", kind, 4, 10, out.data_ptr(), _lib.stream_of(out))
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
