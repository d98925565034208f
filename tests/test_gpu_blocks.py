"""The refiner block (configs 4-5) on the HIP ops vs the same composition on the oracle, with the block's packed
weights and calibrated static scales: the depthwise producer, the chained-quant-out expand and the residual contract.
Tolerance is for the whole block: each of three quantization steps may flip codes where the FP32 accumulation order
differs, so relative L2 <= 1e-2 (MXFP8) / 2e-2 (INT8) of the output and per-stage checks in test_gpu_conv /
test_gpu_depthwise carry the per-op contracts."""

import pytest
import torch

from flashim_amd import blocks
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _oracle_block(block: blocks.RefinerBlock, x: torch.Tensor) -> torch.Tensor:
    b, h, w, c = x.shape
    dw_w, dw_b = block.dw_weight.cpu(), block.dw_bias.cpu()
    xn = x.permute(0, 3, 1, 2)
    one = (1, 1, 1, 1, 0, 0, 1, 1)
    if block.preset == "mxfp8":
        e1, e2 = block.in_scale.cpu(), block.hidden_scale.cpu()
        q1 = ref.depthwise5x5_gelu(xn, dw_w, dw_b, exponent=e1).view(b, h, w, c)
        q2 = ref.mxfp8_conv2d(q1, e1, block.w1.values.cpu(), block.w1.scale_exponent.cpu(), block.b1.cpu(), *one,
                              gelu=True, out_exponent=e2)
        return ref.mxfp8_conv2d(q2, e2, block.w2.values.cpu(), block.w2.scale_exponent.cpu(), block.b2.cpu(), *one,
                                residual=x)
    s1, s2 = block.in_scale.cpu(), block.hidden_scale.cpu()
    q1 = ref.depthwise5x5_gelu(xn, dw_w, dw_b, scale=s1).view(b, h, w, c)
    q2 = ref.int8_conv2d(q1, block.w1_q.cpu(), s1, block.w1_s.cpu(), block.b1.cpu(), *one, gelu=True, out_scale=s2)
    return ref.int8_conv2d(q2, block.w2_q.cpu(), s2, block.w2_s.cpu(), block.b2.cpu(), *one, residual=x)


@pytest.mark.parametrize("preset,tol", [("mxfp8", 1e-2), ("int8", 2e-2)])
@pytest.mark.parametrize("channels,hw", [(64, (40, 37)), (128, (16, 20))])
def test_refiner_block_matches_oracle(preset, tol, channels, hw):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, *hw, channels, generator=g).to(torch.bfloat16)
    block = blocks.RefinerBlock(blocks.BlockWeights.random(channels, g, DEV), preset).calibrate(x.to(DEV))
    got = block(x.to(DEV)).cpu().float()
    want = _oracle_block(block, x).float()
    assert got.shape == want.shape == (2, *hw, channels)
    rel = ((got - want).norm() / want.norm()).item()
    assert rel <= tol, rel
    # the residual path alone is exact structure: output minus input is the block's contribution
    assert torch.isfinite(got).all()


def test_stack_runs_and_is_deterministic():
    scales = blocks.build_stack("mxfp8", DEV)
    # shrink: only the coarsest scale for the test
    first = blocks.run_stack(scales[:1])
    again = blocks.run_stack(scales[:1])
    assert all(torch.equal(a, b) for a, b in zip(first, again))


def test_stack_two_streams_matches_serial():
    """The directions on two streams give the serial stack's bits, eagerly and in every replay of a captured graph
    (replayed several times with eager work and synchronizations in between)."""
    scales = blocks.build_stack("mxfp8", DEV)[:2]  # the two coarsest scales
    side = torch.cuda.Stream()
    want = blocks.run_stack(scales)
    got = blocks.run_stack(scales, side)
    torch.cuda.synchronize()
    assert len(got) == len(want) and all(torch.equal(a, b) for a, b in zip(got, want))
    graph = torch.cuda.CUDAGraph()
    blocks.run_stack(scales, side)  # warm-up outside the capture
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        captured = blocks.run_stack(scales, side)
    for _ in range(3):
        eager = blocks.run_stack(scales)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(captured, eager))
