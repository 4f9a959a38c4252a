"""plh_forward_noalloc: the allocation-free variant of plh_forward (device scratch inside the
library instead of a caller workspace), called through the C ABI.  Checked against plh_forward
(bit for bit: same kernels, same launch plan) and against the CPU oracle, on two calls in a row, the
second smaller (it then runs on scratch still holding the first call's data); its status word read
with plh_noalloc_status; one call captured in a HIP graph and replayed several times with eager
work between the replays (a plh_forward and a smaller plh_forward_noalloc that overwrites the shared
scratch), each replay bit for bit against plh_forward; and its rejection of a forward that needs
more scratch than it holds or has negative sizes."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import assert_close, linear_params, make_regressor, make_x, oracle_layers
from oracle import oracle

pytestmark = pytest.mark.gpu

PLH_ERR_INVALID = 1


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _noalloc_status(gpu):
    st = ctypes.c_uint32(0xFFFFFFFF)
    rc = gpu.lib.plh_noalloc_status(ctypes.byref(st), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, gpu.last_error()
    return st.value


def _noalloc(gpu, blob, dims, x, probes, outs):
    I, H, L, O = dims
    B, T = int(x.size(0)), int(x.size(1))
    pd = torch.tensor(probes, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    return gpu.lib.plh_forward_noalloc(
        blob.data_ptr(), I, H, L, O, x.data_ptr(), B, T, None, None, None, outs["out"].data_ptr(),
        outs["out_seq"].data_ptr(), outs["h_n"].data_ptr(), outs["c_n"].data_ptr(), pd.data_ptr(), len(probes),
        outs["probe_h"].data_ptr(), outs["probe_c"].data_ptr(), stream)


@pytest.mark.parametrize("first,second", [((5, 128, 4, 24, 48, 300), (5, 128, 2, 7, 9, 40)),
                                          ((5, 256, 2, 6, 40, 64), (3, 100, 3, 5, 5, 17))])
def test_noalloc_matches_plh_forward_twice(gpu, first, second):
    assert gpu.lib.plh_noalloc_scratch_bytes() == 64 << 20
    for I, H, L, O, B, T in (first, second):
        _say(f"noalloc I={I} H={H} L={L} O={O} B={B} T={T}")
        native = make_regressor(I, H, L, O)
        x = make_x(B, T, I)
        xd = x.to("cuda", torch.float16).contiguous()
        blob = gpu.pack(*[[getattr(native.lstm, f"{n}_l{l}").detach().cuda() for l in range(L)]
                          for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")],
                        native.linear.weight.detach().cuda(), native.linear.bias.detach().cuda())
        probes = [1, T // 2, T]
        ref = gpu.forward(blob, (I, H, L, O), xd, want_seq=True, want_state=True, probe_steps=probes,
                          check_status=True)
        outs = {k: torch.full_like(v, 7.0) for k, v in ref.items()}
        rc = _noalloc(gpu, blob, (I, H, L, O), xd, probes, outs)
        assert rc == 0, gpu.last_error()
        assert _noalloc_status(gpu) == 0, "the noalloc forward's own status word reports a failed wait"
        torch.cuda.synchronize()
        for k in ref:
            assert torch.equal(outs[k], ref[k]), f"{k} differs from plh_forward"
        want = oracle.regressor_forward(x.numpy(), oracle_layers(native.lstm), *linear_params(native.linear))
        assert_close(outs["out"].float().cpu().numpy(), want, what="noalloc head vs oracle")


def test_noalloc_rejects_a_forward_larger_than_its_scratch(gpu):
    _say("noalloc oversize")
    I, H, L, O, B, T = 5, 128, 4, 24, 512, 1000
    need = gpu.workspace_bytes(I, H, L, O, B, T)
    assert need > 64 << 20
    blob = torch.zeros(gpu.packed_bytes(I, H, L, O), dtype=torch.uint8, device="cuda")
    x = torch.zeros(B, T, I, dtype=torch.float16, device="cuda")
    outs = {"out": torch.full((B, O), 7.0, dtype=torch.float16, device="cuda"),
            "out_seq": torch.full((1,), 7.0, dtype=torch.float16, device="cuda"),
            "h_n": torch.full((1,), 7.0, dtype=torch.float16, device="cuda"),
            "c_n": torch.full((1,), 7.0, dtype=torch.float16, device="cuda"),
            "probe_h": torch.full((1,), 7.0, device="cuda"), "probe_c": torch.full((1,), 7.0, device="cuda")}
    stream = torch.cuda.current_stream().cuda_stream
    rc = gpu.lib.plh_forward_noalloc(blob.data_ptr(), I, H, L, O, x.data_ptr(), B, T, None, None, None,
                                     outs["out"].data_ptr(), None, None, None, None, 0, None, None, stream)
    assert rc == PLH_ERR_INVALID
    assert "MiB of device scratch" in gpu.last_error()
    torch.cuda.synchronize()
    assert (outs["out"] == 7.0).all(), "nothing may be launched for a rejected forward"


def test_noalloc_rejects_negative_sizes(gpu):
    _say("noalloc negative sizes")
    for B, T in ((-1, 10), (4, -1)):
        rc = gpu.lib.plh_forward_noalloc(None, 5, 128, 4, 24, None, B, T, None, None, None, None, None, None, None,
                                         None, 0, None, None, None)
        assert rc == PLH_ERR_INVALID, (B, T, rc)
        assert "non-negative" in gpu.last_error()


def _call(gpu, blob, dims, x, pd, n_probe, outs):
    I, H, L, O = dims
    return gpu.lib.plh_forward_noalloc(
        blob.data_ptr(), I, H, L, O, x.data_ptr(), int(x.size(0)), int(x.size(1)), None, None, None,
        outs["out"].data_ptr(), outs["out_seq"].data_ptr(), outs["h_n"].data_ptr(), outs["c_n"].data_ptr(),
        pd.data_ptr(), n_probe, outs["probe_h"].data_ptr(), outs["probe_c"].data_ptr(),
        torch.cuda.current_stream().cuda_stream)


def _setup(gpu, I, H, L, O, B, T, seed):
    native = make_regressor(I, H, L, O)
    xd = make_x(B, T, I, seed=seed).to("cuda", torch.float16).contiguous()
    blob = gpu.pack(*[[getattr(native.lstm, f"{n}_l{l}").detach().cuda() for l in range(L)]
                      for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")],
                    native.linear.weight.detach().cuda(), native.linear.bias.detach().cuda())
    probes = [1, T // 2, T]
    ref = gpu.forward(blob, (I, H, L, O), xd, want_seq=True, want_state=True, probe_steps=probes, check_status=True)
    outs = {k: torch.full_like(v, 7.0) for k, v in ref.items()}
    pd = torch.tensor(probes, dtype=torch.int32, device="cuda")
    return blob, xd, ref, outs, pd


@pytest.mark.parametrize("dims,B,T", [((5, 128, 4, 24), 48, 200), ((5, 256, 2, 6), 32, 64)])
def test_noalloc_replays_in_a_hip_graph(gpu, dims, B, T):
    I, H, L, O = dims
    _say(f"noalloc graph I={I} H={H} L={L} O={O} B={B} T={T}")
    blob, xd, ref, outs, pd = _setup(gpu, I, H, L, O, B, T, seed=1)
    # the eager work between replays: a smaller forward of the same model
    x2 = make_x(B // 4, T // 3, I, seed=5).to("cuda", torch.float16).contiguous()
    ref2 =gpu.forward(blob, dims, x2, want_seq=True, want_state=True, probe_steps=[1, (T // 3) // 2, T // 3],
                       check_status=True)
    outs2 = {k: torch.full_like(v, 7.0) for k, v in ref2.items()}
    pd2 = torch.tensor([1, (T // 3) // 2, T // 3], dtype=torch.int32, device="cuda")

    # One eager call first (looks up the scratch address and the occupancy outside the capture).
    assert _call(gpu, blob, dims, xd, pd, 3, outs) == 0, gpu.last_error()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _call(gpu, blob, dims, xd, pd, 3, outs)
    assert rc == 0, gpu.last_error()
    torch.cuda.synchronize()
    for rep in range(4):
        for v in outs.values():
            v.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert _noalloc_status(gpu) == 0, f"replay {rep}: status word set"
        for k in ref:
            assert torch.equal(outs[k], ref[k]), f"replay {rep}: {k} differs from plh_forward"
        # eager work between replays: plh_forward of another input, and a smaller noalloc forward that
        # leaves its own data in the shared scratch
        other = gpu.forward(blob, dims, x2, want_seq=True, want_state=True, probe_steps=[1, (T // 3) // 2, T // 3])
        for v in outs2.values():
            v.fill_(7.0)
        assert _call(gpu, blob, dims, x2, pd2, 3, outs2) == 0, gpu.last_error()
        torch.cuda.synchronize()
        assert _noalloc_status(gpu) == 0
        for k in ref2:
            assert torch.equal(outs2[k], ref2[k]), f"eager noalloc after replay {rep}: {k}"
            assert torch.equal(other[k], ref2[k]), f"eager plh_forward after replay {rep}: {k}"
    del graph
