"""plh_forward_noalloc under HIP graph capture: one allocation-free forward captured in a graph and
replayed several times, with eager work between the replays (a plh_forward and a smaller
plh_forward_noalloc that overwrites the shared scratch), each replay checked bit for bit against
plh_forward's eager result and its status word read with plh_noalloc_status."""
from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import make_regressor, make_x

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _status(gpu):
    st = ctypes.c_uint32(0xFFFFFFFF)
    rc = gpu.lib.plh_noalloc_status(ctypes.byref(st), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, gpu.last_error()
    return st.value


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
        assert _status(gpu) == 0, f"replay {rep}: status word set"
        for k in ref:
            assert torch.equal(outs[k], ref[k]), f"replay {rep}: {k} differs from plh_forward"
        # eager work between replays: plh_forward of another input, and a smaller noalloc forward that
        # leaves its own data in the shared scratch
        other = gpu.forward(blob, dims, x2, want_seq=True, want_state=True, probe_steps=[1, (T // 3) // 2, T // 3])
        for v in outs2.values():
            v.fill_(7.0)
        assert _call(gpu, blob, dims, x2, pd2, 3, outs2) == 0, gpu.last_error()
        torch.cuda.synchronize()
        assert _status(gpu) == 0
        for k in ref2:
            assert torch.equal(outs2[k], ref2[k]), f"eager noalloc after replay {rep}: {k}"
            assert torch.equal(other[k], ref2[k]), f"eager plh_forward after replay {rep}: {k}"
    del graph
