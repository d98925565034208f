"""CPU tests of everything but the GPU compute: the C-ABI library loads and exports every symbol the header declares,
the host build of the kernels' scalar numerics matches torch exhaustively, the dispatcher's selection rules
(priority, when / accepts, pins and FLASHIM_OPS overrides, bind / prepare, profiler ranges), platform detection, the
no-fallback rule, and the host-side layout / packing helpers."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from flashim_amd import _lib, blocks, dispatch, ops, quant
from flashim_amd.platforms import Feature, Platform, rocm_features
from oracle import reference as ref

ROOT = Path(__file__).resolve().parents[1]


# -- the C ABI ---------------------------------------------------------------------------------------------------


def test_library_exports_every_declared_symbol():
    header = (ROOT / "include" / "flashim_amd.h").read_text()
    declared = set(re.findall(r"^int (fim_\w+)\(", header, re.M))
    assert {"fim_int8_conv2d", "fim_mxfp8_conv2d", "fim_quantize_mxfp8", "fim_depthwise5x5"} <= declared
    lib = _lib.load()
    for name in declared:
        assert hasattr(lib, name), name
    assert declared <= set(_lib.SIGNATURES), "every declared entry point has a ctypes signature"
    assert lib.fim_version() >= 100


def test_probes_live_in_their_own_library():
    """The test / measurement hooks are built into libflashim_amd_probe.so, not the product library or its header."""
    header = (ROOT / "include" / "flashim_amd.h").read_text()
    assert "fim_test_" not in header
    probe_header = (ROOT / "flashim_amd" / "csrc" / "probe.h").read_text()
    declared = set(re.findall(r"^int (fim_\w+)\(", probe_header, re.M))
    assert declared == set(_lib.PROBE_SIGNATURES)
    probe, lib = _lib.load_probe(), _lib.load()
    for name in declared:
        assert hasattr(probe, name), name
        with pytest.raises(AttributeError):
            getattr(lib, name)


def test_header_compiles_as_c():
    import subprocess

    src = '#include "flashim_amd.h"\nint main(void) { return fim_version == 0; }\n'
    r = subprocess.run(["gcc", "-x", "c", "-std=c99", "-fsyntax-only", f"-I{ROOT / 'include'}", "-"],
                       input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_argument_errors_are_reported_without_a_gpu():
    lib = _lib.load()
    # null pointers are rejected before any launch
    assert lib.fim_quantize_int8(None, 1, 1, 1, 1, 8, 8, 8, 8, 1, None, None, None, None) == _lib.FIM_ERR_INVALID
    assert lib.fim_mxfp8_conv2d(*([None] + [1] * 4 + [None] * 2 + [1] + [None] * 2 + [0] + [1] * 10 + [None, 0, 0,
                                None, None, None, None])) == _lib.FIM_ERR_INVALID
    with pytest.raises(_lib.UnsupportedShape):
        _lib.check(99, "x")
    with pytest.raises(RuntimeError, match="code 7"):
        _lib.check(7, "x")


def test_depthwise_rejects_channel_counts_past_its_32_bit_indexing():
    lib = _lib.load()
    fake = 1 << 20  # 16-byte aligned stand-ins: the call must return before touching memory or launching
    c = 85899360  # a multiple of 32 above INT32_MAX / 25 (the weight index (ky * 5 + kx) * C + c)
    assert lib.fim_depthwise5x5(fake, 1, 1, 1, c, fake, fake, 0, 0, 2, None, None, fake, None, None,
                                None) == _lib.FIM_ERR_UNSUPPORTED
    assert lib.fim_depthwise5x5(fake, 1 << 20, 1 << 10, 1 << 10, 32, fake, fake, 0, 0, 2, None, None, fake, None, None,
                                None) == _lib.FIM_ERR_UNSUPPORTED  # 2^45 elements
    assert lib.fim_depthwise5x5(fake, 1, 1, 1, 32, fake, fake, 2, 0, 2, None, None, fake, None, None,
                                None) == _lib.FIM_ERR_INVALID  # bias dtype code


def test_int8_linear_quantize_rejects_a_row_stride_below_n():
    lib = _lib.load()
    fake = 1 << 20
    assert lib.fim_int8_linear_quantize(fake, 4, 32, fake, 16, fake, None, fake, None, 0, fake, fake, 8,
                                        None) == _lib.FIM_ERR_INVALID


def test_noalloc_calibration_rejects_widths_past_its_scratch_without_a_gpu():
    lib = _lib.load()
    fake = 1 << 20
    assert lib.fim_calibrate_block32_noalloc(fake, 0, 1, 131073, 131073, fake, None) == _lib.FIM_ERR_UNSUPPORTED
    assert lib.fim_calibrate_block32_noalloc(None, 0, 1, 32, 32, fake, None) == _lib.FIM_ERR_INVALID
    assert lib.fim_calibrate_block32_noalloc(fake, 7, 1, 32, 32, fake, None) == _lib.FIM_ERR_UNSUPPORTED


# -- host build of the scalar numerics ---------------------------------------------------------------------------


def _host():
    return _lib.load_host()


def _call(fn, x: np.ndarray, out_dtype, *extra):
    x = np.ascontiguousarray(x)
    out = np.empty(x.size, dtype=out_dtype)
    fn(x.ctypes.data_as(ctypes.c_void_p), ctypes.c_int64(x.size), *extra, out.ctypes.data_as(ctypes.c_void_p))
    return out


def test_host_e4m3_encoder_matches_torch():
    h = _host()
    bf = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    bf = bf[torch.isfinite(bf)].clamp(-448, 448)
    torch.manual_seed(0)
    rnd = (torch.randn(1 << 20) * torch.exp2(torch.randint(-25, 10, (1 << 20,)).float())).clamp(-448, 448)
    for x in (bf, rnd):
        got = _call(h.fim_host_e4m3, x.numpy().astype(np.float32), np.uint8)
        assert np.array_equal(got, x.to(torch.float8_e4m3fn).view(torch.uint8).numpy())
    codes = np.arange(256, dtype=np.uint8)
    dec = _call(h.fim_host_e4m3_decode, codes, np.float32)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    finite = np.isfinite(want)
    assert np.array_equal(dec[finite], want[finite]) and np.isnan(dec[~finite]).all()


def test_host_mx_exponent_matches_torch_at_every_power_of_two_boundary():
    h = _host()
    torch.manual_seed(0)
    ks = torch.arange(-149, 128).double()
    bnd = (torch.exp2(ks)[:, None] * (1 + torch.arange(0, 64).double()[None] * 2.0**-23) * 448).float().flatten()
    amax = torch.cat([torch.tensor([0.0, 448, 449, 1, 1e-30, 1e-45]), bnd, bnd.nextafter(torch.tensor(0.0)),
                      bnd.nextafter(torch.tensor(3e38)),
                      torch.rand(1 << 18) * torch.exp2(torch.randint(-140, 120, (1 << 18,)).float())])
    amax = amax[torch.isfinite(amax)]
    got = _call(h.fim_host_mx_exponent, amax.numpy(), np.int8)
    assert np.array_equal(got, ref.scale_exponent_from_amax(amax).numpy())


def test_host_mx_exponent_fast_path_matches_torch():
    """The division-free exponent (amax * RN(1/448), decided from the product's bits away from powers of two) gives
    torch's exponent wherever it decides, at every power-of-two boundary and its neighbours and on random amax; it
    declines zero, subnormal quotients and the few units around each power of two, and decides almost every random
    value."""
    h = _host()
    torch.manual_seed(1)
    ks = torch.arange(-149, 128).double()
    steps = torch.cat([torch.arange(0, 64), (1 << 23) - torch.arange(1, 64)]).double()
    bnd = (torch.exp2(ks)[:, None] * (1 + steps[None] * 2.0**-23) * 448).float().flatten()
    rnd = torch.rand(1 << 20) * torch.exp2(torch.randint(-140, 120, (1 << 20,)).float())
    amax = torch.cat([torch.tensor([0.0, 448, 449, 1, 1e-30, 1e-45, 3.4e38]), bnd, bnd.nextafter(torch.tensor(0.0)),
                      bnd.nextafter(torch.tensor(3e38)), rnd])
    amax = amax[torch.isfinite(amax)].contiguous()
    x = amax.numpy()
    out = np.empty(x.size, np.int8)
    decided = np.empty(x.size, np.uint8)
    h.fim_host_mx_exponent_fast(x.ctypes.data_as(ctypes.c_void_p), ctypes.c_int64(x.size),
                                out.ctypes.data_as(ctypes.c_void_p), decided.ctypes.data_as(ctypes.c_void_p))
    assert np.array_equal(out, ref.scale_exponent_from_amax(amax).numpy())
    assert decided[:7].tolist() == [0, 0, 1, 1, 1, 0, 1]  # zero, 448 = 448 x 2^0 and 2^-149 decline
    tail = decided[-rnd.numel():][rnd.numpy() > 1e-30]  # below 448 x 2^-126 the quotient is subnormal
    assert tail.mean() > 0.999, tail.mean()


def test_host_bf16_and_int8_rounding_match_torch():
    h = _host()
    torch.manual_seed(0)
    x = torch.randn(1 << 18) * torch.exp2(torch.randint(-30, 30, (1 << 18,)).float())
    got = _call(h.fim_host_bf16, x.numpy(), np.uint16)
    assert np.array_equal(got, x.to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16))
    y = torch.randn(1 << 18) * 40
    got = _call(h.fim_host_quantize_int8, y.numpy(), np.int8, ctypes.c_float(0.37))
    assert np.array_equal(got, ref.quantize_int8_static(y, torch.tensor(0.37)).numpy())


# -- the dispatcher ----------------------------------------------------------------------------------------------


def _toy_op(name):
    dispatch.OPS.pop(name, None)
    op = dispatch.Op(name)
    cpu = dispatch.DeviceSpec("cpu")
    op.register("low", device=cpu, priority=0)(lambda x: ("low", x))
    op.register("high", device=cpu, priority=1, when=lambda x: x > 0)(lambda x: ("high", x))
    op.register("optin", device=cpu, priority=-1)(lambda x: ("optin", x))
    op.register("rocm", device=dispatch.DeviceSpec("rocm"), requires=[Feature.HIP])(lambda x: ("rocm", x))
    return op


def test_dispatch_order_when_optin_and_pins():
    op = _toy_op("toy_dispatch")
    t = torch.tensor(1.0)
    assert op(t)[0] == "high"
    assert op(-t)[0] == "low"  # when() refuses -> next impl
    assert op.get("optin")(t)[0] == "optin"  # negative priority: only pinned
    with pytest.raises(NotImplementedError, match="when"):
        op.get("high")(-t)  # a pinned impl that does not apply raises: there is no fallback
    report = op.explain(-t)
    assert report["low"] == "selected" and report["high"] == "when() refused the arguments"
    assert report["rocm"].startswith("registered for rocm") and report["optin"].startswith("opt-in")
    assert op.supports(t) and op.get(None) is op
    with pytest.raises(ValueError):
        op.get("missing")
    with pytest.raises(ValueError):
        op.register("low", device=dispatch.DeviceSpec("cpu"))


@pytest.mark.parametrize("wildcard_first", [True, False])
def test_dispatch_ties_prefer_the_narrower_device_spec(wildcard_first):
    """Equal priority: the platform-specific impl beats a '*' impl whatever the registration order, as FlashIM's
    registry sorts by (priority, capability span, order) (flashim/ops/_registry.py:62-68, 214)."""
    name = f"toy_span_{wildcard_first}"
    dispatch.OPS.pop(name, None)
    op = dispatch.Op(name)
    specs = [("any", dispatch.DeviceSpec("*")), ("cpu", dispatch.DeviceSpec("cpu"))]
    for impl, spec in (specs if wildcard_first else specs[::-1]):
        op.register(impl, device=spec, priority=1)(lambda x, impl=impl: impl)
    op.register("narrow", device=dispatch.DeviceSpec("cpu"), priority=0)(lambda x: "narrow")
    assert op(torch.tensor(1.0)) == "cpu"
    assert [e.name for e in op.impls] == ["cpu", "any", "narrow"]  # priority still decides first
    assert dispatch.DeviceSpec("*").span == float("inf")
    assert dispatch.DeviceSpec("cuda", (8, 0), (9, 0)).span == 100.0 < dispatch.DeviceSpec("cuda").span


def test_dispatch_overrides_and_counts():
    op = _toy_op("toy_overrides")
    t = torch.tensor(1.0)
    dispatch.configure("toy_overrides:low")
    assert op(t)[0] == "low"
    dispatch.configure("-toy_overrides")
    with pytest.raises(NotImplementedError, match="switched off"):
        op(t)
    assert not op.supports(t)
    dispatch.configure(None)
    with pytest.raises(ValueError):
        dispatch.configure("bogus")
    dispatch.reset_call_counts()
    op(t), op(-t)
    assert dispatch.call_counts()["toy_overrides"] == {"high": 1, "low": 1}


def test_dispatch_profiler_range_names_op_and_impl():
    op = _toy_op("toy_range")
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU]) as prof:
        op(torch.tensor(1.0))
    assert any(e.name == "flashim::toy_range[high]" for e in prof.events())


def test_dispatch_bind_prepares_once():
    dispatch.OPS.pop("toy_bind", None)
    op = dispatch.Op("toy_bind", weights=1)
    calls = []
    op.register("packed", device=dispatch.DeviceSpec("cpu"),
                prepare=lambda w: (calls.append(1) or w * 10,))(lambda x, w: x + w)
    op.register("plain", device=dispatch.DeviceSpec("cpu"), priority=-1)(lambda x, w: x - w)
    bound = op.bind(torch.tensor(1.0)).warmup()
    assert bound.primary == "packed" and bound.available == ["packed"] and len(calls) == 1
    assert bound(torch.tensor(2.0)).item() == 12.0 and bound(torch.tensor(3.0)).item() == 13.0
    assert len(calls) == 1
    assert op.bind(torch.tensor(1.0), impl="plain")(torch.tensor(5.0)).item() == 4.0
    with pytest.raises(ValueError):
        op.bind()


def test_platform_features():
    assert rocm_features("gfx950") >= {Feature.HIP, Feature.MFMA_I8, Feature.MFMA_F8F6F4_SCALED, Feature.FP8_E4M3}
    assert Feature.HIP not in rocm_features("gfx942")  # other AMD architectures never select the gfx950 kernels
    p = Platform("rocm", 0, arch="gfx942", features=rocm_features("gfx942"))
    assert not dispatch.DeviceSpec("cuda").matches(p) and dispatch.DeviceSpec("rocm").matches(p)


def test_ops_have_no_cpu_fallback():
    """The product path computes only on the HIP kernels: on a CPU tensor every op refuses loudly."""
    x = torch.randint(-127, 127, (1, 4, 4, 16), dtype=torch.int8)
    w = torch.randint(-127, 127, (8, 9 * 16), dtype=torch.int8)
    with pytest.raises(NotImplementedError, match="no HIP impl"):
        ops.int8_conv2d(x, w, torch.tensor(0.1), torch.ones(8), None, 3, 3, 1, 1, 1, 1, 1, 1)
    with pytest.raises(NotImplementedError):
        ops.quantize_mxfp8(torch.randn(4, 32), torch.zeros(1, dtype=torch.int8))
    with pytest.raises(RuntimeError, match="GPU only"):
        quant.quantize_static(torch.randn(4, 32), torch.zeros(1, dtype=torch.int8))
    assert ops.int8_conv2d.explain(x, w, torch.tensor(0.1), torch.ones(8), None, 3, 3, 1, 1, 1, 1, 1, 1)["hip"]


# -- host-side layout and packing helpers ------------------------------------------------------------------------


@pytest.mark.parametrize("rows,groups", [(1, 1), (300, 32), (130, 5)])
def test_swizzle_layout_helpers_match_oracle(rows, groups):
    e = torch.randint(-20, 10, (rows, groups), dtype=torch.int8)
    sw = quant.swizzle_scales(e)
    assert torch.equal(sw.view(torch.uint8), ref.swizzle_scales(e))
    assert torch.equal(quant.unswizzle_scales(sw, rows, groups), e)
    assert quant.swizzled_size(rows, groups) == sw.numel()


def test_block_batchnorm_fold_matches_torch_fusion():
    g = torch.Generator().manual_seed(0)
    wts = blocks.BlockWeights.random(32, g, "cpu")
    conv = torch.nn.Conv2d(32, 32, 5, padding=2, groups=32).eval()
    bn = torch.nn.BatchNorm2d(32, eps=blocks.BN_EPS).eval()
    with torch.no_grad():
        conv.weight.copy_(wts.dw_weight), conv.bias.copy_(wts.dw_bias)
        bn.weight.copy_(wts.bn_gamma), bn.bias.copy_(wts.bn_beta)
        bn.running_mean.copy_(wts.bn_mean), bn.running_var.copy_(wts.bn_var)
    fused = torch.nn.utils.fusion.fuse_conv_bn_eval(conv, bn)
    packed, bias = wts.folded_depthwise()
    want = fused.weight.detach()[:, 0].permute(1, 2, 0).reshape(25, 32).to(torch.bfloat16)
    assert torch.equal(packed, want)
    assert torch.allclose(bias, fused.bias.detach(), rtol=1e-6, atol=1e-7)
    x = torch.randn(1, 32, 6, 7)
    assert torch.allclose(F.conv2d(x, fused.weight, fused.bias, padding=2, groups=32), bn(conv(x)), atol=1e-5)
