"""The time-parallel input-projection GEMM (plh_input_projection) against a float64 matmul of the same
fp16 operands.  Floating point: the bound is the fp16 rounding of the result (half an ulp, 2^-11
relative) plus fp32 accumulation error, written below as rtol 2^-10 on |x| |w| row sums."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _check(got: torch.Tensor, x: torch.Tensor, w: torch.Tensor, what: str) -> None:
    xd, wd = x.double().cpu().numpy(), w.double().cpu().numpy()
    want = xd @ wd.T
    scale = np.abs(xd) @ np.abs(wd).T  # bound on the accumulated magnitude
    g = got.double().cpu().numpy()
    err = np.abs(g - want)
    bound = 2.0 ** -10 * np.abs(want) + 2.0 ** -20 * scale + 1e-7
    bad = err > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} entries out of bound, worst {float((err - bound).max()):.3e}"


@pytest.mark.parametrize("M,K,N,pad", [
    (1000, 128, 512, 0),      # the C2 layer shape (K = H = 128), partial m-tile
    (3000, 512, 2048, 0),     # the C4 layer shape, partial m-tile
    (257, 128, 128, 64),      # smallest N; x rows wider than K (ldx > K)
    (5, 384, 1024, 128),      # fewer rows than one tile; K = 300 padded to 384 in a 512-wide buffer
    (70000, 256, 384, 0),     # m-groups with several tiles each at a width of three slices
    (3000, 640, 512, 0),      # K > 512: W held in K blocks of 512 and 128, reloaded per m-tile
    (1100, 1024, 4096, 0),    # the H 1024 layer shape: two K blocks of 512
    (600, 2048, 256, 128),    # four K blocks, x rows wider than K
])
def test_input_projection_matches_float64(gpu, M, K, N, pad):
    print(f"[gpu-case] input projection M={M} K={K} N={N} pad={pad}", flush=True)
    g = torch.Generator().manual_seed(M + K + N)
    x = torch.randn(M, K + pad, generator=g).half()
    w = (torch.rand(N, K, generator=g) * 2 - 1).half() / 8
    xd, wd = x.cuda(), w.cuda()
    got = gpu.input_projection(xd[:, :K], wd)
    torch.cuda.synchronize()
    _check(got, x[:, :K], w, f"M={M} K={K} N={N}")


@pytest.mark.parametrize("M,K,N,ldx", [
    (512000, 512, 2048, 512),  # the C4 layer shape in the layer-sequential path's layout
    (4000, 128, 512, 128),     # the C2 layer shape
    (1616, 384, 2048, 512),    # H = 300 padded to 384 within a 512-wide layer buffer; 101 row blocks
    (128000, 1024, 4096, 1024),  # the H 1024 layer shape of one 128-row launch, T = 1000 (two K blocks)
    (1040, 256, 384, 256),     # 65 row blocks: the last tile's waves hold 1 and 0 valid blocks
    (5008, 512, 1024, 1024),   # x rows wider than K (NaN past K), a partial last tile
    (16, 128, 128, 128),       # a single row block
])
def test_input_projection_blocked_layout(gpu, M, K, N, ldx):
    """Fragment-blocked x and out (the layout the layer-sequential path keeps): the result equals the
    row-major product after from_blocked.  At M = 512000 only rows of the first, a middle and the last
    512-row tile are compared on the host."""
    print(f"[gpu-case] blocked input projection M={M} K={K} N={N} ldx={ldx}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M + K)
    x = torch.randn(M, ldx, device="cuda", generator=g).half()
    x[:, K:] = float("nan")  # columns past K must not be read
    w = (torch.randn(N, K, device="cuda", generator=g) / 16).half()
    xb = gpu.to_blocked(x)
    assert torch.equal(gpu.from_blocked(xb).nan_to_num(7.0), x.nan_to_num(7.0))
    ob = gpu.input_projection(xb, w, blocked=True)
    rows = torch.cat([torch.arange(0, 512), torch.arange(M // 2, M // 2 + 512), torch.arange(M - 512, M)]) \
        if M > 4096 else torch.arange(M)
    got = gpu.from_blocked(ob)[rows.cuda()]
    torch.cuda.synchronize()
    _check(got, x[rows.cuda(), :K].cpu(), w.cpu(), f"blocked M={M}")


def test_input_projection_output_stride_and_repeat(gpu):
    """Output into a strided view (ldo > N) leaves the other columns alone; two calls agree bitwise."""
    print("[gpu-case] input projection strided out", flush=True)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(600, 128, generator=g).half().cuda()
    w = (torch.randn(256, 128, generator=g) / 16).half().cuda()
    big = torch.full((600, 512), 3.0, dtype=torch.float16, device="cuda")
    gpu.input_projection(x, w, out=big[:, 128:384])
    again = gpu.input_projection(x, w)
    torch.cuda.synchronize()
    assert torch.equal(big[:, 128:384], again)
    assert (big[:, :128] == 3.0).all() and (big[:, 384:] == 3.0).all()
    _check(again, x.cpu(), w.cpu(), "strided")


def test_input_projection_rejects_bad_shapes(gpu):
    def z(*shape):
        return torch.zeros(*shape, dtype=torch.float16, device="cuda")
    for xs, ws in (((10, 96), (256, 96)), ((10, 128), (200, 128)), ((10, 650), (256, 650))):
        with pytest.raises(ValueError, match="k % 128"):
            gpu.input_projection(z(*xs), z(*ws))
