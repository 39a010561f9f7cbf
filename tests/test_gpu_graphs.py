"""HIP-graph capture of the ops: a captured call keeps the workspace and scratch addresses it was
captured with, so the pools must keep those buffers alive when a later, larger call grows them
(kernelbench_harbor_amd/ops.py _WorkspacePool). Between replays the test grows the pools with a
larger eager call and allocates tensors that would land on a freed buffer; each replay must
match the eager result and leave those tensors untouched."""
import pytest
import torch

from kernelbench_harbor_amd import inputs, ops

pytestmark = pytest.mark.gpu


def _capture(fn, args):
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        fn(*args)                       # warm-up on the capture stream (sizes its pools)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        out = fn(*args)
    return g, st, out


@pytest.mark.parametrize("op", ["w4a16_decode", "w4a16_wide", "w8a8", "mxfp8_dma"])
def test_replay_after_pool_growth(dev, op):
    print(f"[graph] {op}", flush=True)
    if op == "w4a16_decode":      # split-K workspace
        small = [t.to(dev) for t in inputs.w4a16(16, 2048, 512, seed=1)]
        big = [t.to(dev) for t in inputs.w4a16(16, 14336, 4096, seed=2)]
        fn = ops.w4a16_gemm
    elif op == "w4a16_wide":      # split-K scratch of the wide-tile kernel
        small = [t.to(dev) for t in inputs.w4a16(64, 2048, 512, seed=3)]
        big = [t.to(dev) for t in inputs.w4a16(64, 14336, 4096, seed=4)]
        fn = ops.w4a16_gemm
    elif op == "mxfp8_dma":       # split-K workspace of the 256 x 256 LDS-DMA tiles
        small = [t.to(dev) for t in inputs.mxfp8(1024, 1024, 256, seed=7)]
        big = [t.to(dev) for t in inputs.mxfp8(2048, 14336, 4096, seed=8)]
        fn = ops.mxfp8_gemm
    else:
        small = [t.to(dev) for t in inputs.w8a8(16, 2048, 512, seed=5)]
        big = [t.to(dev) for t in inputs.w8a8(16, 14336, 4096, seed=6)]
        fn = ops.w8a8_gemm
    g, st, out = _capture(fn, small)
    want = fn(*small).clone()
    for rep in range(3):
        with torch.cuda.stream(st):
            fn(*big)                     # grows the pools of this stream (first time)
            junk = [torch.full((1 << 22,), 7.0, device=dev) for _ in range(8)]
            g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
        assert all(bool((j == 7.0).all()) for j in junk), rep   # nobody else's memory written
        del junk
    del g
