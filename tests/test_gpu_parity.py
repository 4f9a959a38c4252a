"""Parity of the HIP forward against the CPU oracle (oracle/lstm_oracle.c) and torch's fp32 nn.LSTM.

Bar: max-abs <= 2e-2 and mean-abs <= 2e-3 on the [B, O] output, and the same
bound on every layer's h and c after 1, 100 and 1000 steps.  The GPU runs fp16 weights (a .half()
copy of the seeded fp32 model); the references run the original fp32 weights.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import (assert_close, linear_params, make_lengths, make_regressor, make_x, oracle_layers)
from oracle import oracle
from persistent_lstm_hip_amd import PersistentLSTM, PersistentLSTMRegressor, convert_regressor_module

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _gpu_model(native):
    m = PersistentLSTMRegressor.from_native_module(native).to("cuda").half().eval()
    return m


def _torch_ref(native, x, lengths=None):
    with torch.inference_mode():
        if lengths is None:
            return native(x).numpy()
        packed = torch.nn.utils.rnn.pack_padded_sequence(x, lengths, batch_first=True, enforce_sorted=False)
        _, (h, _) = native.lstm(packed)
        return native.linear(h[-1]).numpy()


@pytest.mark.parametrize("I,H,L,O,B,T", [
    (5, 128, 1, 24, 8, 64),      # C1 shape
    (5, 32, 2, 7, 20, 37),       # H bucket 32, ragged tile, T not a multiple of the chunk
    (5, 64, 3, 24, 33, 19),      # H bucket 64
    (17, 100, 2, 5, 16, 9),      # padded H and I > 8
    (5, 128, 4, 24, 48, 130),    # headline geometry, small batch
    (5, 256, 2, 24, 20, 37),     # sliced: 4 workgroups per (layer, tile), ragged tile
    (5, 200, 3, 5, 33, 19),      # sliced, padded H in the 256 bucket
    (5, 512, 2, 24, 16, 21),     # sliced: 16 workgroups per (layer, tile)
    (37, 300, 2, 3, 18, 11),     # sliced, padded H in the 512 bucket, I > 32
])
def test_regressor_matches_oracle(gpu, I, H, L, O, B, T):
    _say(f"regressor I={I} H={H} L={L} O={O} B={B} T={T}")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I)
    want = oracle.regressor_forward(x.numpy(), oracle_layers(native.lstm), *linear_params(native.linear))
    np.testing.assert_allclose(want, _torch_ref(native, x), atol=1e-5)
    got = _gpu_model(native)(x.to("cuda", torch.float16))
    gpu.check_status(torch.device("cuda"))
    assert got.dtype == torch.float16 and tuple(got.shape) == (B, O)
    assert_close(got.float().cpu().numpy(), want, what="out")


def test_headline_c2_full_batch(gpu):
    """C2: 4 layers, H128, B512, T1000.  Full output vs torch fp32 CPU; probes vs the oracle."""
    I, H, L, O, B, T = 5, 128, 4, 24, 512, 1000
    _say("C2 full batch")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I)
    model = _gpu_model(native)
    xg = x.to("cuda", torch.float16)
    out, ph, pc = model.forward_probe(xg, [1, 100, 1000])
    gpu.check_status(torch.device("cuda"))
    out2 = model(xg)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "probe and plain forward disagree"
    want = _torch_ref(native, x)
    mx, mn = assert_close(out.float().cpu().numpy(), want, what="C2 out vs torch fp32")
    _say(f"C2 out vs torch fp32: max_abs={mx:.3e} mean_abs={mn:.3e}")
    rows = np.r_[0:16, 250:266, 496:512]
    ref = oracle.lstm_forward(x.numpy()[rows], oracle_layers(native.lstm), probe_steps=(1, 100, 1000))
    for p, step in enumerate((1, 100, 1000)):
        for name, got_all, want_all in (("h", ph, ref["probe_h"]), ("c", pc, ref["probe_c"])):
            g = got_all[p][:, rows].cpu().numpy()
            mx, mn = assert_close(g, want_all[p], what=f"{name} after {step} steps")
            _say(f"{name}@{step}: max_abs={mx:.3e} mean_abs={mn:.3e}")


def test_ragged_c5(gpu):
    """C5: lengths ~ U[200, 1000] sorted descending, packed-sequence semantics, head on h_n[-1]."""
    I, H, L, O, B, T = 5, 128, 4, 24, 512, 1000
    _say("C5 ragged")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I)
    lengths = make_lengths(B, T, 200)
    model = _gpu_model(native)
    out = model.forward_ragged(x.to("cuda", torch.float16), lengths)
    gpu.check_status(torch.device("cuda"))
    want = _torch_ref(native, x, lengths)
    mx, mn = assert_close(out.float().cpu().numpy(), want, what="C5 out vs packed torch")
    _say(f"C5 vs packed torch: max_abs={mx:.3e} mean_abs={mn:.3e}")
    rows = np.r_[0:16, 300:316, 496:512]
    ref = oracle.regressor_forward(x.numpy()[rows], oracle_layers(native.lstm), *linear_params(native.linear),
                                   lengths=lengths.numpy()[rows])
    assert_close(out.float().cpu().numpy()[rows], ref, what="C5 out vs oracle")


def test_ragged_small_unsorted_with_zero_length(gpu):
    I, H, L, O, B, T = 5, 64, 2, 3, 21, 40
    _say("ragged small unsorted")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I)
    lengths = torch.randint(1, T + 1, (B,), generator=torch.Generator().manual_seed(5))
    lengths[3] = 0
    lengths[7] = T
    model = _gpu_model(native)
    got = model.forward_ragged(x.to("cuda", torch.float16), lengths).float().cpu().numpy()
    want = oracle.regressor_forward(x.numpy(), oracle_layers(native.lstm), *linear_params(native.linear),
                                    lengths=lengths.numpy())
    assert_close(got, want, what="ragged small")
    # a zero-length row never updates: the head sees h = 0
    np.testing.assert_allclose(got[3], native.linear.bias.detach().numpy(), atol=2e-3)


def test_ragged_length_sources_and_back_to_back_calls(gpu):
    """Lengths as a list, a strided host tensor and a device tensor give the same result, and
    back-to-back calls with different host lengths (staged through pinned memory without a stream
    synchronisation) each see their own lengths."""
    I, H, L, O, B, T = 5, 128, 3, 6, 40, 48
    _say("ragged length sources")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I)
    xd = x.to("cuda", torch.float16)
    model = _gpu_model(native)
    g = torch.Generator().manual_seed(11)
    wide = torch.randint(0, T + 1, (2 * B,), generator=g)
    base = wide[::2]  # strided host tensor
    assert not base.is_contiguous()
    want = oracle.regressor_forward(x.numpy(), oracle_layers(native.lstm), *linear_params(native.linear),
                                    lengths=base.numpy())
    for src in (base.tolist(), base, base.to("cuda")):
        got = model.forward_ragged(xd, src).float().cpu().numpy()
        assert_close(got, want, what=f"lengths from {type(src).__name__}")
    sets = [torch.randint(1, T + 1, (B,), generator=g) for _ in range(4)]
    outs = [model.forward_ragged(xd, s) for s in sets]  # no synchronisation between the calls
    for s, o in zip(sets, outs):
        ref = oracle.regressor_forward(x.numpy(), oracle_layers(native.lstm), *linear_params(native.linear),
                                       lengths=s.numpy())
        assert_close(o.float().cpu().numpy(), ref, what="back-to-back ragged call")
    gpu.check_status(torch.device("cuda"))


def test_persistent_lstm_dropin(gpu):
    I, H, L, B, T = 5, 128, 2, 24, 50
    _say("PersistentLSTM drop-in")
    torch.manual_seed(7)
    lstm = torch.nn.LSTM(I, H, L, batch_first=True).eval()
    x = make_x(B, T, I, seed=3)
    g = torch.Generator().manual_seed(4)
    h0 = 0.5 * torch.randn(L, B, H, generator=g)
    c0 = 0.5 * torch.randn(L, B, H, generator=g)
    with torch.inference_mode():
        want_out, (want_h, want_c) = lstm(x, (h0, c0))
    mod = PersistentLSTM.from_native_module(lstm).to("cuda").half()
    out, (h, c) = mod(x.to("cuda", torch.float16), (h0.cuda().half(), c0.cuda().half()))
    gpu.check_status(torch.device("cuda"))
    assert tuple(out.shape) == (B, T, H) and tuple(h.shape) == (L, B, H)
    assert_close(out.float().cpu().numpy(), want_out.numpy(), what="out seq")
    assert_close(h.float().cpu().numpy(), want_h.numpy(), what="h_n")
    assert_close(c.float().cpu().numpy(), want_c.numpy(), what="c_n")
    # PackedSequence input
    lengths = torch.tensor(sorted(torch.randint(1, T + 1, (B,), generator=g).tolist(), reverse=True))
    packed = torch.nn.utils.rnn.pack_padded_sequence(x, lengths, batch_first=True)
    with torch.inference_mode():
        wp, (wh, wc) = lstm(packed)
    wpad, _ = torch.nn.utils.rnn.pad_packed_sequence(wp, batch_first=True, total_length=T)
    gp = torch.nn.utils.rnn.pack_padded_sequence(x.to("cuda", torch.float16), lengths, batch_first=True)
    op, (oh, oc) = mod(gp)
    opad, _ = torch.nn.utils.rnn.pad_packed_sequence(op, batch_first=True, total_length=T)
    assert_close(opad.float().cpu().numpy(), wpad.numpy(), what="packed out")
    assert_close(oh.float().cpu().numpy(), wh.numpy(), what="packed h_n")
    assert_close(oc.float().cpu().numpy(), wc.numpy(), what="packed c_n")


def test_row_permutation_and_determinism(gpu):
    I, H, L, O, B, T = 5, 128, 4, 24, 64, 200
    _say("permutation + determinism")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I).to("cuda", torch.float16)
    model = _gpu_model(native)
    a = model(x)
    b = model(x)
    perm = torch.randperm(B, generator=torch.Generator().manual_seed(9)).cuda()
    c = model(x[perm])
    torch.cuda.synchronize()
    assert torch.equal(a, b), "two runs differ"
    assert torch.equal(a[perm], c), "batch rows are not independent"


def test_uniform_batch_shortcut(gpu):
    I, H, L, O, B, T = 5, 128, 4, 24, 512, 300
    _say("uniform batch")
    native = make_regressor(I, H, L, O)
    model = _gpu_model(native)
    x = torch.ones(B, T, I, device="cuda", dtype=torch.float16)
    out = model(x)
    torch.cuda.synchronize()
    assert torch.equal(out, out[:1].expand_as(out))
    want = _torch_ref(native, torch.ones(1, T, I))
    assert_close(out[:1].float().cpu().numpy(), want, what="uniform row")


def test_reference_extension_surface(gpu):
    """The reference's extension entry points, fed the reference's packed formats."""
    I, H, L, O, B, T = 5, 128, 4, 24, 32, 60
    _say("extension surface")
    native = make_regressor(I, H, L, O).to("cuda").half()
    x = make_x(B, T, I).to("cuda", torch.float16)
    lstm = native.lstm

    def kpairs(w):  # P[p, c, j] = W[c, 2p + j], zero-padded to even K
        k = w.shape[1]
        wt = torch.nn.functional.pad(w.t(), (0, 0, 0, k % 2))
        return wt.reshape(-1, 2, w.shape[0]).permute(0, 2, 1).contiguous()

    fused = [getattr(lstm, f"bias_ih_l{l}") + getattr(lstm, f"bias_hh_l{l}") for l in range(L)]
    w_ih = [getattr(lstm, f"weight_ih_l{l}") for l in range(L)]
    w_hh = [getattr(lstm, f"weight_hh_l{l}") for l in range(L)]
    want = convert_regressor_module(native)(x)
    a = gpu.persistent_lstm_regressor_forward_generic_projected(x, w_ih, w_hh, fused, native.linear.weight,
                                                                native.linear.bias)
    args = []
    for l in range(L):
        args += [kpairs(w_ih[l]), kpairs(w_hh[l]), fused[l]]
    b = gpu.persistent_lstm4_forward_interleaved(x, *args, native.linear.weight, native.linear.bias)
    r = gpu.repeat_first_row(a[:1], 7)
    torch.cuda.synchronize()
    # the reference fuses the bias in fp16 before the kernel: allow that rounding
    assert_close(a.float().cpu().numpy(), want.float().cpu().numpy(), max_abs=2e-3, mean_abs=5e-4, what="generic")
    assert torch.equal(a, b)
    assert torch.equal(r, a[:1].expand(7, -1))


@pytest.mark.parametrize("B,T", [(600, 120), (2100, 40)])
def test_large_batches_use_16_row_tiles_and_split_launches(gpu, B, T):
    """600 rows need 16-row tiles to fit one co-resident launch; 2100 rows need several launches."""
    I, H, L, O = 5, 128, 4, 24
    _say(f"large batch B={B} T={T}")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I)
    model = _gpu_model(native)
    got = model(x.to("cuda", torch.float16))
    gpu.check_status(torch.device("cuda"))
    want = _torch_ref(native, x)
    assert_close(got.float().cpu().numpy(), want, what=f"B={B}")
    rows = np.r_[0:8, B // 2:B // 2 + 8, B - 8:B]
    ref = oracle.regressor_forward(x.numpy()[rows], oracle_layers(native.lstm), *linear_params(native.linear))
    assert_close(got.float().cpu().numpy()[rows], ref, what=f"B={B} vs oracle")


@pytest.mark.parametrize("H,L,B,T", [
    (256, 4, 200, 60),    # sliced, 13 tiles x 4 layers = 52 groups: grid rounded up to 56
    (256, 3, 400, 30),    # sliced, two tiles per workgroup, 13 tile groups x 3 layers = 39 -> 40
    (512, 2, 48, 40),     # sliced at H 512, 3 tiles x 2 layers = 6 groups -> 8
    (512, 2, 320, 30),    # layer-sequential, 20 tiles -> 24
    (1000, 2, 200, 12),   # layer-sequential at padded H 1024, 13 tiles: launches of 8 and 5 -> 8
])
def test_grids_rounded_up_to_whole_xcds(gpu, H, L, B, T):
    """Batches whose tile (or tile group) count is not a multiple of 8 launch a grid rounded up to one,
    whose extra workgroups return at once: every row against torch fp32, rows at both ends and the
    middle against the oracle, and the extra workgroups leave the status word clear."""
    I, O = 5, 16
    _say(f"rounded-up grid H={H} L={L} B={B} T={T}")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I)
    got = _gpu_model(native)(x.to("cuda", torch.float16))
    gpu.check_status(torch.device("cuda"))
    assert_close(got.float().cpu().numpy(), _torch_ref(native, x), what=f"H={H} B={B}")
    rows = np.r_[0:4, B // 2:B // 2 + 4, B - 4:B]
    ref = oracle.regressor_forward(x.numpy()[rows], oracle_layers(native.lstm), *linear_params(native.linear))
    assert_close(got.float().cpu().numpy()[rows], ref, what=f"H={H} B={B} vs oracle")


@pytest.mark.parametrize("H", [256, 512])
def test_large_hidden_c3_c4(gpu, H):
    """C3 (H256) and C4 (H512): 4 layers, B512, T1000.  C3 runs the sliced kernel (two tiles per
    workgroup), C4 the layer-sequential path (one 512-row launch per layer).

    Output vs torch fp32 on all 512 rows; h and c of every layer after 1, 100 and 1000 steps vs the
    oracle on 32 rows spread over the batch (every tile group and both ends).
    """
    I, L, O, B, T = 5, 4, 24, 512, 1000
    _say(f"large hidden H={H} B={B} T={T}")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I)
    model = _gpu_model(native)
    out, ph, pc = model.forward_probe(x.to("cuda", torch.float16), [1, 100, 1000])
    gpu.check_status(torch.device("cuda"))
    want = _torch_ref(native, x)
    mx, mn = assert_close(out.float().cpu().numpy(), want, what=f"H={H} out vs torch fp32 (all {B} rows)")
    _say(f"H={H} out vs torch fp32: max_abs={mx:.3e} mean_abs={mn:.3e}")
    prow = np.unique(np.r_[0:4, np.linspace(4, B - 5, 24).astype(int), B - 4:B])
    assert prow.size >= 32
    ref = oracle.lstm_forward(x.numpy()[prow], oracle_layers(native.lstm), probe_steps=(1, 100, 1000))
    for p, step in enumerate((1, 100, 1000)):
        for name, got_all, want_all in (("h", ph, ref["probe_h"]), ("c", pc, ref["probe_c"])):
            g = got_all[p][:, prow].cpu().numpy()
            mx, mn = assert_close(g, want_all[p], what=f"H={H} {name} after {step} steps")
            _say(f"H={H} {name}@{step}: max_abs={mx:.3e} mean_abs={mn:.3e}")


@pytest.mark.parametrize("I,H,L,O,B,T,ragged,state", [
    (5, 600, 2, 3, 20, 30, False, False),     # padded H 1024, layer 0 projected inside the kernel
    (5, 1024, 2, 24, 150, 12, True, True),    # H 1024, two launches of 128 + 22 rows, ragged, h0/c0
    (300, 256, 2, 6, 33, 20, False, True),    # I > H: layer by layer at padded H 256, GEMM K 384
    (300, 1024, 2, 5, 16, 15, True, False),   # H 1024 with a GEMM-projected layer 0 (K 384)
    (1000, 600, 1, 3, 18, 12, False, False),  # I 1000: GEMM K 1024 (two K blocks), x in its own buffer
    (600, 700, 2, 7, 24, 10, False, True),    # K 640: a K block of 512 and one of 128
    (70, 50, 3, 4, 30, 25, True, False),      # H 50 < I 70: padded to 128, layer by layer
    (33, 32, 2, 4, 17, 21, False, False),     # H 32 < I 33
    (40, 520, 1, 2, 300, 6, False, False),    # H 520, three launches of 128 rows
])
def test_wide_hidden_and_input_against_oracle(gpu, I, H, L, O, B, T, ragged, state):
    """The reference's generic entry point serves 1 <= H <= 1024 and any input size
    (model.py:154-165, persistent_lstm_hip.cu:2981-2991).  Here H 513..1024 and inputs wider than the
    padded hidden size run the layer-sequential path (projection GEMM + W_hh-only persistent kernel);
    every output (head, sequence, final h/c, probed h/c) against the C oracle at the north-star
    tolerance, and the path's own rounding (ref_fp16_proj, or ref_fp16_proj_l1 where layer 0 is
    projected in the kernel) within the regression bounds."""
    _say(f"wide I={I} H={H} L={L} O={O} B={B} T={T} ragged={ragged} state={state}")
    assert gpu.supports(I, H, L, O)
    torch.manual_seed(1000 + H + I)
    lstm = torch.nn.LSTM(I, H, L, batch_first=True)
    head = torch.nn.Linear(H, O)
    x = torch.randn(B, T, I, generator=torch.Generator().manual_seed(H))
    g = torch.Generator().manual_seed(I)
    lengths = torch.randint(0, T + 1, (B,), generator=g) if ragged else None
    h0 = (0.5 * torch.randn(L, B, H, generator=g)).half() if state else None
    c0 = (0.5 * torch.randn(L, B, H, generator=g)).half() if state else None
    probes = [1, max(1, T // 2), T]
    params = [[getattr(lstm, f"{n}_l{l}").detach().cuda() for l in range(L)]
              for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
    packed = gpu.pack(*params, head.weight.detach().cuda(), head.bias.detach().cuda())
    dev = torch.device("cuda")
    res = gpu.forward(packed, (I, H, L, O), x.to(dev, torch.float16), lengths=lengths,
                      h0=None if h0 is None else h0.to(dev), c0=None if c0 is None else c0.to(dev),
                      want_seq=True, want_state=True, probe_steps=probes, check_status=True)
    kw = dict(lengths=None if lengths is None else lengths.numpy(), h0=None if h0 is None else h0.float().numpy(),
              c0=None if c0 is None else c0.float().numpy(), probe_steps=probes, want_seq=True)
    want = oracle.lstm_forward(x.numpy(), oracle_layers(lstm), **kw)
    tag = f"I={I} H={H}"
    for k in ("out_seq", "h_n", "c_n", "probe_h", "probe_c"):
        mx, mn = assert_close(res[k].float().cpu().numpy(), want[k], what=f"{tag} {k}")
    w_head = oracle.linear(want["h_n"][-1], *linear_params(head))
    mx, mn = assert_close(res["out"].float().cpu().numpy(), w_head, what=f"{tag} head")
    _say(f"{tag}: head max_abs {mx:.2e} mean_abs {mn:.2e}")
    # (every case here runs layer by layer: padded H 1024, or an input above the padded H; layer 0 is
    # projected inside the kernel, in fp32, when I <= 32)
    numerics = "ref_fp16_proj_l1" if (I <= 32 and H > 512) else "ref_fp16_proj"
    ref = oracle.lstm_forward(x.numpy(), oracle_layers(lstm), numerics=numerics, **kw)
    # a flipped fp16 rounding of a large input projection (I up to 1000) moves a gate by up to half an
    # fp16 ulp of it: the bound is 20x below the north star's
    for k, bound in (("probe_h", 1e-3), ("probe_c", 1e-3)):
        assert_close(res[k].float().cpu().numpy(), ref[k], max_abs=bound, mean_abs=bound / 10,
                     what=f"{tag} {k} vs {numerics}")


def test_generic_projected_entry_point_at_h1024(gpu):
    """persistent_lstm_hip_ext.persistent_lstm_regressor_forward_generic_projected (bindings.cpp:163) at
    H = 1024 with the reference's argument formats (torch-layout W_ih/W_hh lists, fp16 fused biases),
    against the oracle fed the same fp16 values."""
    import persistent_lstm_hip_ext as ext_mod

    I, H, L, O, B, T = 5, 1024, 2, 24, 40, 20
    _say("generic_projected H=1024")
    native = make_regressor(I, H, L, O).half()
    dev = torch.device("cuda")
    w_ih = [getattr(native.lstm, f"weight_ih_l{l}").detach().to(dev) for l in range(L)]
    w_hh = [getattr(native.lstm, f"weight_hh_l{l}").detach().to(dev) for l in range(L)]
    fused = [(getattr(native.lstm, f"bias_ih_l{l}") + getattr(native.lstm, f"bias_hh_l{l}")).detach().to(dev)
             for l in range(L)]
    lw, lb = native.linear.weight.detach().to(dev), native.linear.bias.detach().to(dev)
    x = make_x(B, T, I).half()
    got = ext_mod.persistent_lstm_regressor_forward_generic_projected(x.to(dev), w_ih, w_hh, fused, lw, lb)
    layers = [(w_ih[l].float().cpu().numpy(), w_hh[l].float().cpu().numpy(), fused[l].float().cpu().numpy(), None)
              for l in range(L)]
    want = oracle.regressor_forward(x.float().numpy(), layers, lw.float().cpu().numpy(), lb.float().cpu().numpy())
    mx, mn = assert_close(got.float().cpu().numpy(), want, what="generic_projected H=1024")
    _say(f"generic_projected H=1024: max_abs {mx:.2e} mean_abs {mn:.2e}")


def test_h512_row_pinned_on_both_paths(gpu):
    """At padded H 512 the batch size picks the path (L = 4: B <= 256 the all-layers sliced kernel,
    whose projections stay fp32; B > 256 the layer-sequential path, whose GEMM projections of layers
    1-3 are fp16).  The same rows at B = 256 and B = 320 are each pinned to the oracle's restatement
    of their own rounding (ref_fp16 / ref_fp16_proj_l1) with the regression bounds, and both to the
    fp32 oracle at the north-star tolerance."""
    I, H, L, O, T = 5, 512, 4, 24, 300
    native = make_regressor(I, H, L, O)
    model = _gpu_model(native)
    x = make_x(320, T, I)
    rows = np.r_[0:6, 250:256]
    layers = oracle_layers(native.lstm)
    lw, lb = linear_params(native.linear)
    want32 = oracle.regressor_forward(x.numpy()[rows], layers, lw, lb)
    got = {}
    for B, numerics in ((256, "ref_fp16"), (320, "ref_fp16_proj_l1")):
        _say(f"H512 pinned rows at B={B} ({numerics})")
        out, ph, pc = model.forward_probe(x[:B].to("cuda", torch.float16), [T])
        gpu.check_status(torch.device("cuda"))
        got[B] = out.float().cpu().numpy()[rows]
        ref = oracle.lstm_forward(x.numpy()[rows], layers, numerics=numerics, probe_steps=(T,))
        head = oracle.linear(ref["h_n"][-1], lw, lb, numerics="ref_fp16")
        mx, mn = assert_close(got[B], head, max_abs=2e-4, mean_abs=2e-5, what=f"B={B} head vs {numerics}")
        _say(f"B={B} head vs {numerics}: max_abs {mx:.2e}")
        for name, g, w in (("h", ph, ref["probe_h"]), ("c", pc, ref["probe_c"])):
            assert_close(g[0][:, rows].cpu().numpy(), w[0], max_abs=4e-4, mean_abs=4e-5, what=f"B={B} {name}")
        assert_close(got[B], want32, what=f"B={B} head vs fp32 oracle")
    assert not np.array_equal(got[256], got[320]), "the two paths are expected to round differently"


def test_sliced_persistent_lstm_dropin_with_state(gpu):
    """H256 PersistentLSTM with h0/c0, full output sequence and final state, plus ragged lengths."""
    I, H, L, B, T = 24, 256, 2, 40, 33
    _say("sliced PersistentLSTM drop-in")
    torch.manual_seed(11)
    lstm = torch.nn.LSTM(I, H, L, batch_first=True).eval()
    x = make_x(B, T, I, seed=12)
    g = torch.Generator().manual_seed(13)
    h0 = 0.5 * torch.randn(L, B, H, generator=g)
    c0 = 0.5 * torch.randn(L, B, H, generator=g)
    with torch.inference_mode():
        want_out, (want_h, want_c) = lstm(x, (h0, c0))
    mod = PersistentLSTM.from_native_module(lstm).to("cuda").half()
    out, (h, c) = mod(x.to("cuda", torch.float16), (h0.cuda().half(), c0.cuda().half()))
    gpu.check_status(torch.device("cuda"))
    assert_close(out.float().cpu().numpy(), want_out.numpy(), what="sliced out seq")
    assert_close(h.float().cpu().numpy(), want_h.numpy(), what="sliced h_n")
    assert_close(c.float().cpu().numpy(), want_c.numpy(), what="sliced c_n")
    lengths = torch.tensor(sorted(torch.randint(0, T + 1, (B,), generator=g).tolist(), reverse=True))
    lengths[0] = T
    lengths[-1] = 0
    native = make_regressor(I, H, L, 6)
    model = _gpu_model(native)
    got = model.forward_ragged(x.to("cuda", torch.float16), lengths).float().cpu().numpy()
    want = oracle.regressor_forward(x.numpy(), oracle_layers(native.lstm), *linear_params(native.linear),
                                    lengths=lengths.numpy())
    assert_close(got, want, what="sliced ragged")


@pytest.mark.parametrize("H", [512, 300])
def test_layer_sequential_path_dropin_with_state_and_ragged(gpu, H):
    """H512-bucket batches that need several wavefront launches run layer by layer (input projection
    as one fp16 GEMM per layer, then the W_hh-only recurrent kernel): 1100 rows are three launches of
    up to 512 rows.  PersistentLSTM with h0/c0, the full output sequence and the final state vs torch
    fp32; then ragged lengths (zeros included, unsorted) through the regressor vs the oracle."""
    I, L, B, T = 24, 2, 1100, 7
    _say(f"layer-sequential H={H} B={B} T={T}")
    torch.manual_seed(31)
    lstm = torch.nn.LSTM(I, H, L, batch_first=True).eval()
    x = make_x(B, T, I, seed=32)
    g = torch.Generator().manual_seed(33)
    h0 = 0.5 * torch.randn(L, B, H, generator=g)
    c0 = 0.5 * torch.randn(L, B, H, generator=g)
    with torch.inference_mode():
        want_out, (want_h, want_c) = lstm(x, (h0, c0))
    mod = PersistentLSTM.from_native_module(lstm).to("cuda").half()
    out, (h, c) = mod(x.to("cuda", torch.float16), (h0.cuda().half(), c0.cuda().half()))
    gpu.check_status(torch.device("cuda"))
    assert_close(out.float().cpu().numpy(), want_out.numpy(), what="layer-sequential out seq")
    assert_close(h.float().cpu().numpy(), want_h.numpy(), what="layer-sequential h_n")
    assert_close(c.float().cpu().numpy(), want_c.numpy(), what="layer-sequential c_n")
    lengths = torch.randint(0, T + 1, (B,), generator=g)
    lengths[5] = 0
    lengths[700] = T
    native = make_regressor(I, H, L, 6)
    model = _gpu_model(native)
    got = model.forward_ragged(x.to("cuda", torch.float16), lengths).float().cpu().numpy()
    gpu.check_status(torch.device("cuda"))
    rows = np.r_[0:40, 500:530, 1060:1100]  # every launch, the partial last one included
    want = oracle.regressor_forward(x.numpy()[rows], oracle_layers(native.lstm), *linear_params(native.linear),
                                    lengths=lengths.numpy()[rows])
    assert_close(got[rows], want, what="layer-sequential ragged")


@pytest.mark.parametrize("T", [1, 2, 3])
def test_layer_sequential_short_sequences(gpu, T):
    """Layer-sequential path with 1, 2 and 3 steps (the kernel loads each step's projection a step
    ahead, clamped to the last step): 600 rows are a 512-row launch and an 88-row one (6 tiles, no
    XCD mapping, so agent-scope exchange).  Full output sequence and final state vs torch fp32."""
    I, H, L, B = 5, 512, 2, 600
    _say(f"layer-sequential short T={T}")
    torch.manual_seed(41)
    lstm = torch.nn.LSTM(I, H, L, batch_first=True).eval()
    x = make_x(B, T, I, seed=42)
    g = torch.Generator().manual_seed(43)
    h0 = 0.5 * torch.randn(L, B, H, generator=g)
    c0 = 0.5 * torch.randn(L, B, H, generator=g)
    with torch.inference_mode():
        want_out, (want_h, want_c) = lstm(x, (h0, c0))
    mod = PersistentLSTM.from_native_module(lstm).to("cuda").half()
    out, (h, c) = mod(x.to("cuda", torch.float16), (h0.cuda().half(), c0.cuda().half()))
    gpu.check_status(torch.device("cuda"))
    assert_close(out.float().cpu().numpy(), want_out.numpy(), what=f"T={T} out seq")
    assert_close(h.float().cpu().numpy(), want_h.numpy(), what=f"T={T} h_n")
    assert_close(c.float().cpu().numpy(), want_c.numpy(), what=f"T={T} c_n")


@pytest.mark.parametrize("H,B,T", [(512, 600, 2), (256, 600, 5), (256, 40, 5), (512, 200, 3)],
                         ids=["layer-sequential", "sliced-two-tiles", "sliced-one-tile", "sliced-H512"])
def test_packed_exchange_zero_lengths_large_state_and_nan(gpu, H, B, T):
    """The layer-sequential and sliced exchanges pack 4 fp16 per word with the step tag in bit 14 of
    each (clear in every computed h).  Rows of length 0 keep h0, which may use that bit (|h0| >= 2
    here): their results must still be exact, and no wait may hang on a clobbered tag.  A NaN input
    row must give NaN (NaN travels as a reserved code) and leave the other rows untouched.  At L = 2
    the path follows from the batch: H512 with 600 rows runs layer by layer, H512 with 200 rows and
    H256 run the sliced kernel (600 rows: two tiles per workgroup; 40 rows: one)."""
    I, L, O = 5, 2, 7
    _say(f"packed exchange zero lengths, |h0| >= 2, NaN row H={H} B={B} T={T}")
    device = torch.device("cuda")
    torch.manual_seed(51)
    lstm = torch.nn.LSTM(I, H, L, batch_first=True)
    head = torch.nn.Linear(H, O)
    x = torch.randn(B, T, I, generator=torch.Generator().manual_seed(52))
    g = torch.Generator().manual_seed(53)
    lengths = torch.randint(0, T + 1, (B,), generator=g)
    lengths[:20] = 0
    lengths[B // 2:B // 2 + 10] = 0
    h0 = (3.0 * torch.randn(L, B, H, generator=g)).half()
    c0 = (0.5 * torch.randn(L, B, H, generator=g)).half()
    params = [[getattr(lstm, f"{n}_l{l}").detach().cuda() for l in range(L)]
              for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
    packed = gpu.pack(*params, head.weight.detach().cuda(), head.bias.detach().cuda())
    res = gpu.forward(packed, (I, H, L, O), x.to(device, torch.float16), lengths=lengths, h0=h0.to(device),
                      c0=c0.to(device), want_out=True, want_seq=True, want_state=True, probe_steps=[1, 2],
                      check_status=True)
    rows = np.unique(np.r_[0:min(40, B), B // 2 - 5:B // 2 + 20, max(0, B - 40):B])
    want = oracle.lstm_forward(x.numpy()[rows], oracle_layers(lstm), lengths=lengths.numpy()[rows],
                               h0=h0.float().numpy()[:, rows], c0=c0.float().numpy()[:, rows],
                               probe_steps=[1, 2], want_seq=True)
    assert_close(res["out_seq"].float().cpu().numpy()[rows], want["out_seq"], what="out_seq")
    assert_close(res["h_n"].float().cpu().numpy()[:, rows], want["h_n"], what="h_n")
    assert_close(res["c_n"].float().cpu().numpy()[:, rows], want["c_n"], what="c_n")
    assert_close(res["probe_h"].cpu().numpy()[:, :, rows], want["probe_h"], what="probe_h")
    w_head = oracle.linear(want["h_n"][-1], *linear_params(head))
    assert_close(res["out"].float().cpu().numpy()[rows], w_head, what="head (h0 rows restored)")
    # a NaN input on one full-length row
    xn = x.clone()
    xn[7, 1, 2] = float("nan")
    full = torch.full((B,), T, dtype=torch.int64)
    res_n = gpu.forward(packed, (I, H, L, O), xn.to(device, torch.float16), lengths=full, want_out=True,
                        want_seq=False, want_state=True, check_status=True)
    res_c = gpu.forward(packed, (I, H, L, O), x.to(device, torch.float16), lengths=full, want_out=True,
                        want_seq=False, want_state=True, check_status=True)
    assert torch.isnan(res_n["out"][7].float()).all() and torch.isnan(res_n["h_n"][:, 7].float()).all()
    others = np.r_[0:7, 8:B]
    np.testing.assert_array_equal(res_n["out"].cpu().numpy()[others], res_c["out"].cpu().numpy()[others])


@pytest.mark.parametrize("H,B", [(128, 16), (256, 16), (256, 600), (512, 600)])
def test_wait_timeout_is_reported_and_recovers(gpu, H, B):
    """A forced 1 us wait bound: the next layer's first hand-off wait cannot be met, so the kernel sets
    the timeout status, poisons the outputs and ends; the front end raises; the default bound then
    gives correct results again (the status word is cleared by every forward).  (256, 600) runs the
    two-tile sliced workgroups, (512, 600) the layer-sequential path.

    Every output element of the timed-out forward - output sequence, final states, probes, head -
    is either NaN (the workgroups whose waits failed poison all their outputs) or its correct value
    (workgroups that completed before the failure); none holds stale memory."""
    I, L, O, T = 5, 2, 3, 64
    _say(f"forced wait timeout H={H} B={B}")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I)
    model = _gpu_model(native)
    xg = x.to("cuda", torch.float16)
    # The layer-sequential path's per-step waits end within microseconds, too soon for any bound:
    # its failure is injected at step 5 instead.
    force = (lambda: gpu.inject_wait_failure(5)) if H == 512 else (lambda: gpu.set_wait_limit(1e-6))
    unforce = (lambda: gpu.inject_wait_failure(None)) if H == 512 else (lambda: gpu.set_wait_limit(None))
    force()
    try:
        out = model(xg)
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError, match="timed out"):
            gpu.check_status(torch.device("cuda"))
        assert torch.isnan(out.float()).any(), "a timed-out forward must poison its outputs"
    finally:
        unforce()
    got = model(xg)
    gpu.check_status(torch.device("cuda"))
    want = oracle.regressor_forward(x.numpy(), oracle_layers(native.lstm), *linear_params(native.linear))
    assert_close(got.float().cpu().numpy(), want, what="after timeout")

    # every requested output of a timed-out forward: NaN or correct (outputs pre-filled with 7.0 so
    # that an element nobody wrote would show)
    blob = model.lstm.packed_blob(xg.device, model.linear)
    ref = oracle.lstm_forward(x.numpy(), oracle_layers(native.lstm), probe_steps=(1, T // 2, T), want_seq=True)
    force()
    try:
        P = 3
        fill = {"out": torch.full((B, O), 7.0, device="cuda", dtype=torch.float16),
                "out_seq": torch.full((B, T, H), 7.0, device="cuda", dtype=torch.float16),
                "h_n": torch.full((L, B, H), 7.0, device="cuda", dtype=torch.float16),
                "c_n": torch.full((L, B, H), 7.0, device="cuda", dtype=torch.float16),
                "probe_h": torch.full((P, L, B, H), 7.0, device="cuda"),
                "probe_c": torch.full((P, L, B, H), 7.0, device="cuda")}
        res = gpu.forward(blob, (I, H, L, O), xg, want_seq=True, want_state=True, probe_steps=(1, T // 2, T),
                          outputs=fill)
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError, match="timed out"):
            gpu.check_status(torch.device("cuda"))
    finally:
        unforce()
    nan_seen = False
    w_head = oracle.linear(ref["h_n"][-1], *linear_params(native.linear))
    for k, w in (("out_seq", ref["out_seq"]), ("h_n", ref["h_n"]), ("c_n", ref["c_n"]), ("probe_h", ref["probe_h"]),
                 ("probe_c", ref["probe_c"]), ("out", w_head)):
        g = res[k].float().cpu().numpy()
        bad = ~np.isnan(g) & (np.abs(g - w) > 2e-2)
        assert not bad.any(), f"{k}: {int(bad.sum())} elements neither NaN nor correct"
        nan_seen |= bool(np.isnan(g).any())
    assert nan_seen, "a timed-out forward must poison the outputs it could not compute"


@pytest.mark.parametrize("I,H,L,O,B,T,zero_tail", [
    (5, 128, 1, 4, 1, 1, False),      # one row, one step
    (128, 128, 2, 4, 9, 17, False),   # input as wide as the padded hidden size
    (5, 256, 1, 4, 3, 5, False),      # sliced kernel with a single layer (no hand-off)
    (5, 512, 2, 4, 100, 9, False),    # sliced, 64-row launches: the second launch is partial
    (5, 256, 2, 4, 20, 12, True),     # sliced: rows 16..19 have length 0, so one tile runs no step
    (5, 128, 3, 4, 20, 12, True),     # wavefront: the same with 8-row tiles
])
def test_edge_geometries(gpu, I, H, L, O, B, T, zero_tail):
    _say(f"edge I={I} H={H} L={L} O={O} B={B} T={T} zero_tail={zero_tail}")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I, seed=21)
    model = _gpu_model(native)
    xg = x.to("cuda", torch.float16)
    if zero_tail:
        lengths = torch.randint(1, T + 1, (B,), generator=torch.Generator().manual_seed(22))
        lengths[16:] = 0
        got = model.forward_ragged(xg, lengths)
        want = oracle.regressor_forward(x.numpy(), oracle_layers(native.lstm), *linear_params(native.linear),
                                        lengths=lengths.numpy())
    else:
        got = model(xg)
        want = oracle.regressor_forward(x.numpy(), oracle_layers(native.lstm), *linear_params(native.linear))
    gpu.check_status(torch.device("cuda"))
    assert_close(got.float().cpu().numpy(), want, what="edge geometry")
    if zero_tail:  # zero steps: the head sees h = 0
        np.testing.assert_allclose(got[16:].float().cpu().numpy(),
                                   np.broadcast_to(native.linear.bias.detach().numpy(), (B - 16, O)), atol=2e-3)


@pytest.mark.parametrize("I,H,L,O,B,T", [
    (5, 128, 64, 3, 20, 6),      # 64 layers (the limit): wavefront, 8-row tiles
    (5, 256, 64, 3, 20, 6),      # 64 layers of 4 slices: one tile fills the device
    (5, 512, 17, 3, 20, 6),      # padded H 512 beyond 16 layers: one tile would not fit the sliced
    (5, 300, 64, 3, 9, 4),       # path, so the layer-sequential path runs it (also at I <= 32, B = 9)
    (5, 64, 2, 4096, 12, 5),     # the largest head
    (65536, 64, 2, 7, 4, 3),     # the largest input: layer 0's projection GEMM over K = 65536
])
def test_limit_geometries(gpu, I, H, L, O, B, T):
    """Geometries at the documented limits (64 layers, head 4096, input 65536) and deep stacks at
    padded H 512, whose tiles only the layer-sequential path can hold, against the oracle."""
    _say(f"limits I={I} H={H} L={L} O={O} B={B} T={T}")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I)
    got = _gpu_model(native)(x.to("cuda", torch.float16))
    gpu.check_status(torch.device("cuda"))
    want = oracle.regressor_forward(x.numpy(), oracle_layers(native.lstm), *linear_params(native.linear))
    assert_close(got.float().cpu().numpy(), want, what="limit geometry out")


@pytest.mark.parametrize("H,B", [(128, 16), (256, 8)])
def test_long_sequence_drift(gpu, H, B):
    """Ten thousand steps (ten times the north star's): h and c of every layer after 1, 5000 and 10000
    steps and the head stay within the bound against the fp32 oracle (fp16 h storage does not
    accumulate into drift)."""
    I, L, O, T = 5, 4, 24, 10000
    _say(f"long sequence H={H} B={B} T={T}")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I)
    model = _gpu_model(native)
    out, ph, pc = model.forward_probe(x.to("cuda", torch.float16), [1, 5000, 10000])
    gpu.check_status(torch.device("cuda"))
    ref = oracle.lstm_forward(x.numpy(), oracle_layers(native.lstm), probe_steps=(1, 5000, 10000))
    for p, step in enumerate((1, 5000, 10000)):
        assert_close(ph[p].cpu().numpy(), ref["probe_h"][p], what=f"h after {step} steps")
        assert_close(pc[p].cpu().numpy(), ref["probe_c"][p], what=f"c after {step} steps")
    want = oracle.linear(ref["h_n"][-1], *linear_params(native.linear))
    assert_close(out.float().cpu().numpy(), want, what="head after 10000 steps")


@pytest.mark.parametrize("H", [128, 512])
def test_empty_batch(gpu, H):
    """An empty batch gives empty outputs of nn.LSTM's shapes and launches nothing that reads x."""
    I, L, O, T = 5, 2, 3, 7
    _say(f"empty batch H={H}")
    native = make_regressor(I, H, L, O)
    x = torch.zeros(0, T, I, device="cuda", dtype=torch.float16)
    out = _gpu_model(native)(x)
    gpu.check_status(torch.device("cuda"))
    assert tuple(out.shape) == (0, O)
    with torch.inference_mode():
        want_seq, (want_h, _) = native.lstm(torch.zeros(0, T, I))
    mod = PersistentLSTM.from_native_module(native.lstm).to("cuda").half()
    seq, (h_n, c_n) = mod(x)
    assert tuple(seq.shape) == tuple(want_seq.shape) and tuple(h_n.shape) == tuple(want_h.shape)
    assert tuple(c_n.shape) == tuple(want_h.shape)


def test_sliced_side_stream_and_determinism(gpu):
    """H512 on a non-default stream (its own workspace) equals the default-stream result bit for bit."""
    I, H, L, O, B, T = 5, 512, 2, 6, 40, 30
    _say("sliced side stream")
    native = make_regressor(I, H, L, O)
    model = _gpu_model(native)
    xg = make_x(B, T, I).to("cuda", torch.float16)
    a = model(xg)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        b = model(xg)
        gpu.check_status(torch.device("cuda"))
    torch.cuda.current_stream().wait_stream(s)
    c = model(xg)
    gpu.check_status(torch.device("cuda"))
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(a, c)


@pytest.mark.parametrize("H,B", [(128, 512), (256, 512), (512, 512)])
def test_forwards_on_two_streams_interleaved(gpu, H, B):
    """Full-device launches enqueued alternately on two streams (each with its own workspace) and
    never synchronised in between: the library orders them (each waits for the other stream's last
    forward), so none ends partly resident and timed out; every result equals the single-stream one
    bit for bit, and both streams' status words are clean.  H512 at B = 512 runs layer by layer."""
    I, L, O, T = 5, 2, 6, 40
    _say(f"two streams H={H} B={B}")
    native = make_regressor(I, H, L, O)
    model = _gpu_model(native)
    xg = make_x(B, T, I).to("cuda", torch.float16)
    ref = model(xg)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    outs = [[], []]
    for _ in range(4):
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                outs[i].append(model(xg))
    for i, st in enumerate(streams):
        with torch.cuda.stream(st):
            gpu.check_status(torch.device("cuda"))
    torch.cuda.synchronize()
    for i in range(2):
        for o in outs[i]:
            assert torch.equal(o, ref), f"stream {i}: result differs from the single-stream forward"


def test_forwards_from_two_host_threads(gpu):
    """Two host threads, each with its own stream, enqueue full-device forwards concurrently (the C
    ABI runs without the GIL): the library's per-device ordering serialises them, and every result
    equals the single-stream one bit for bit."""
    import threading

    I, H, L, O, B, T = 5, 128, 4, 24, 512, 40
    _say("two host threads")
    native = make_regressor(I, H, L, O)
    model = _gpu_model(native)
    xg = make_x(B, T, I).to("cuda", torch.float16)
    ref = model(xg)
    torch.cuda.synchronize()
    outs, errors = [[], []], []

    def work(i):
        try:
            st = torch.cuda.Stream()
            with torch.cuda.stream(st):
                for _ in range(6):
                    outs[i].append(model(xg))
                gpu.check_status(torch.device("cuda"))
            st.synchronize()
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=work, args=(i,)) for i in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in threads), "a forward thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for i in range(2):
        assert len(outs[i]) == 6
        for o in outs[i]:
            assert torch.equal(o, ref), f"thread {i}: result differs from the single-stream forward"


def test_sliced_two_tile_workgroups_ragged_partial_launch(gpu):
    """H256, 4 layers, 600 rows: one-tile workgroups would need several launches, so each workgroup
    carries two software-pipelined tiles (512 rows per launch, then 88 rows with a padding tile), with
    ragged lengths including zeros."""
    I, H, L, O, B, T = 5, 256, 4, 6, 600, 30
    _say(f"sliced two-tile ragged B={B}")
    native = make_regressor(I, H, L, O)
    x = make_x(B, T, I, seed=31)
    lengths = torch.randint(0, T + 1, (B,), generator=torch.Generator().manual_seed(32))
    model = _gpu_model(native)
    got = model.forward_ragged(x.to("cuda", torch.float16), lengths)
    gpu.check_status(torch.device("cuda"))
    want = oracle.regressor_forward(x.numpy(), oracle_layers(native.lstm), *linear_params(native.linear),
                                    lengths=lengths.numpy())
    assert_close(got.float().cpu().numpy(), want, what="two-tile ragged")


def test_mfma_rate_probe(gpu):
    """The roofline constant checked on the box: the probe's dense fp16 MFMA rate is consistent with
    the shader clock it measured (one v_mfma_f32_16x16x32_f16 per 16 cycles per SIMD, 1024 SIMDs)
    and of the order of the published 2.5 PFLOP/s."""
    _say("MFMA rate probe")
    tflops, ghz = gpu.probe_mfma_f16()
    assert 0.5 < ghz < 3.0, ghz
    per_clock = 16 * 16 * 32 * 2 / 16 * 4 * torch.cuda.get_device_properties(0).multi_processor_count
    implied = per_clock * ghz * 1e9 / 1e12
    assert 0.8 * implied < tflops < 1.05 * implied, (tflops, ghz, implied)
    assert 1000.0 < tflops < 3000.0, tflops


def test_kernel_timing_rearm(gpu):
    """plh_kernel_timing: n pairs armed record the next n forwards' persistent launches and no more;
    arming again with the same n re-arms the same events (the warm-up forwards' records are
    discarded), and the times are of the order of the forward's own."""
    _say("kernel timing re-arm")
    native = make_regressor(5, 64, 2, 3)
    model = _gpu_model(native)
    x = make_x(16, 50, 5).to("cuda", torch.float16)
    with torch.inference_mode():
        gpu.kernel_timing(3)
        for _ in range(2):
            model(x)
        gpu.kernel_timing(3)  # re-arm: the two forwards above no longer count
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(5):
            model(x)
        b.record()
        torch.cuda.synchronize()
        ms, n = gpu.kernel_timing_read()
        gpu.kernel_timing(0)
    assert n == 3, n
    assert 0.0 < ms < a.elapsed_time(b), (ms, a.elapsed_time(b))


@pytest.mark.parametrize("seed,count,wide", [(20261203, 64, False), (777, 200, True)])
def test_random_geometry_sweep(gpu, seed, count, wide):
    """Seeded random geometries through plh_forward: input size (also above the padded hidden size),
    hidden size 1..1024 (every kernel family, padded and unpadded), layers, head size (0 = no head),
    batch (above one 128-row launch at padded H 1024), length, ragged lengths with zeros, initial
    states and two probe steps.  Every output (head, sequence, final h/c, probed h/c) is checked
    against the C oracle at the north-star tolerance.  The wide draw also takes batches up to 700
    (several launches, 16-row tiles at H <= 128), sequences up to 260, five layers and inputs up to
    1200."""
    rng = np.random.default_rng(seed)
    device = torch.device("cuda")
    done = 0
    while done < count:
        I = int(rng.integers(1, 41)) if rng.random() < 0.8 else int(rng.integers(41, 1200 if wide else 700))
        u = rng.random()
        H = int(rng.integers(1, 129)) if u < 0.4 else int(rng.integers(129, 513)) if u < 0.75 else \
            int(rng.integers(513, 1025))
        L = int(rng.integers(1, 6 if wide else 5))
        O = 0 if rng.random() < 0.2 else int(rng.integers(1, 31))
        if wide:
            B = int(rng.integers(1, 700)) if H <= 128 else int(rng.integers(1, 330))
            T = int(rng.integers(1, 261))
        else:
            B = int(rng.integers(1, 71)) if H <= 512 else int(rng.integers(1, 161))
            T = int(rng.integers(1, 121))
        if B * T * L * 4 * H * (I + H) > (1e9 if wide else 4e8):
            continue  # keep the oracle to a fraction of a second per case
        ragged = rng.random() < 0.5
        with_state = rng.random() < 0.5
        _say(f"sweep {done}: I={I} H={H} L={L} O={O} B={B} T={T} ragged={ragged} state={with_state}")
        torch.manual_seed(int(rng.integers(1 << 30)))
        lstm = torch.nn.LSTM(I, H, L, batch_first=True)
        head = torch.nn.Linear(H, O) if O else None
        x = torch.randn(B, T, I, generator=torch.Generator().manual_seed(done))
        lengths = torch.tensor(rng.integers(0, T + 1, B), dtype=torch.int64) if ragged else None
        h0 = (0.5 * torch.randn(L, B, H)).half() if with_state else None
        c0 = (0.5 * torch.randn(L, B, H)).half() if with_state else None
        probes = sorted(set(int(p) for p in rng.integers(1, T + 1, 2)))
        params = [[getattr(lstm, f"{n}_l{l}").detach().cuda() for l in range(L)]
                  for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
        packed = gpu.pack(*params, head.weight.detach().cuda() if head else None,
                          head.bias.detach().cuda() if head else None)
        res = gpu.forward(packed, (I, H, L, O), x.to(device, torch.float16), lengths=lengths,
                          h0=None if h0 is None else h0.to(device), c0=None if c0 is None else c0.to(device),
                          want_out=O > 0, want_seq=True, want_state=True, probe_steps=probes, check_status=True)
        want = oracle.lstm_forward(x.numpy(), oracle_layers(lstm), lengths=None if lengths is None else lengths.numpy(),
                                   h0=None if h0 is None else h0.float().numpy(),
                                   c0=None if c0 is None else c0.float().numpy(),
                                   probe_steps=probes, want_seq=True)
        tag = f"sweep {done}"
        assert_close(res["out_seq"].float().cpu().numpy(), want["out_seq"], what=f"{tag} out_seq")
        assert_close(res["h_n"].float().cpu().numpy(), want["h_n"], what=f"{tag} h_n")
        assert_close(res["c_n"].float().cpu().numpy(), want["c_n"], what=f"{tag} c_n")
        assert_close(res["probe_h"].cpu().numpy(), want["probe_h"], what=f"{tag} probe_h")
        assert_close(res["probe_c"].cpu().numpy(), want["probe_c"], what=f"{tag} probe_c")
        if O:
            w_head = oracle.linear(want["h_n"][-1], *linear_params(head))
            assert_close(res["out"].float().cpu().numpy(), w_head, what=f"{tag} head")
        done += 1


@pytest.mark.parametrize("seed,count", [(31, 150)])
def test_random_large_batch_sweep(gpu, seed, count):
    """Seeded random geometries at batch sizes up to 1500 (H <= 128) and 800 (every other H up to
    1024): several launches, 16-row tiles, padded grids and the layer-sequential path at batches the
    whole-batch sweep does not reach.  The GPU runs the whole batch; the oracle runs the first, the
    last and up to 12 other sampled rows (rows are independent), and every output of those rows is
    compared at the north-star tolerance."""
    rng = np.random.default_rng(seed)
    device = torch.device("cuda")
    done = 0
    while done < count:
        I = int(rng.integers(1, 41)) if rng.random() < 0.7 else int(rng.integers(41, 1100))
        u = rng.random()
        H = int(rng.integers(1, 129)) if u < 0.35 else int(rng.integers(129, 513)) if u < 0.75 else \
            int(rng.integers(513, 1025))
        L = int(rng.integers(1, 5))
        O = 0 if rng.random() < 0.15 else int(rng.integers(1, 40))
        B = int(rng.integers(1, 1500)) if H <= 128 else int(rng.integers(1, 800))
        T = int(rng.integers(1, 40)) if rng.random() < 0.7 else int(rng.integers(40, 200))
        rows = np.unique(np.concatenate([rng.choice(B, min(B, 12), replace=False), [0, B - 1]]))
        if len(rows) * T * L * 4 * H * (I + H) > 6e8:
            continue  # keep the oracle to a fraction of a second per case
        ragged = rng.random() < 0.5
        with_state = rng.random() < 0.4
        _say(f"large-batch sweep {done}: I={I} H={H} L={L} O={O} B={B} T={T} ragged={ragged} state={with_state}")
        torch.manual_seed(int(rng.integers(1 << 30)))
        lstm = torch.nn.LSTM(I, H, L, batch_first=True)
        head = torch.nn.Linear(H, O) if O else None
        x = torch.randn(B, T, I, generator=torch.Generator().manual_seed(done))
        lengths = torch.tensor(rng.integers(0, T + 1, B), dtype=torch.int64) if ragged else None
        h0 = (0.5 * torch.randn(L, B, H)).half() if with_state else None
        c0 = (0.5 * torch.randn(L, B, H)).half() if with_state else None
        probes = sorted(set(int(p) for p in rng.integers(1, T + 1, 2)))
        params = [[getattr(lstm, f"{n}_l{l}").detach().cuda() for l in range(L)]
                  for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
        packed = gpu.pack(*params, head.weight.detach().cuda() if head else None,
                          head.bias.detach().cuda() if head else None)
        res = gpu.forward(packed, (I, H, L, O), x.to(device, torch.float16), lengths=lengths,
                          h0=None if h0 is None else h0.to(device), c0=None if c0 is None else c0.to(device),
                          want_out=O > 0, want_seq=True, want_state=True, probe_steps=probes, check_status=True)
        r = torch.from_numpy(rows)
        want = oracle.lstm_forward(x[r].numpy(), oracle_layers(lstm),
                                   lengths=None if lengths is None else lengths[r].numpy(),
                                   h0=None if h0 is None else h0[:, r].float().numpy(),
                                   c0=None if c0 is None else c0[:, r].float().numpy(),
                                   probe_steps=probes, want_seq=True)
        rd = r.to(device)
        tag = f"large-batch sweep {done}"
        assert_close(res["out_seq"][rd].float().cpu().numpy(), want["out_seq"], what=f"{tag} out_seq")
        assert_close(res["h_n"][:, rd].float().cpu().numpy(), want["h_n"], what=f"{tag} h_n")
        assert_close(res["c_n"][:, rd].float().cpu().numpy(), want["c_n"], what=f"{tag} c_n")
        assert_close(res["probe_h"][:, :, rd].cpu().numpy(), want["probe_h"], what=f"{tag} probe_h")
        assert_close(res["probe_c"][:, :, rd].cpu().numpy(), want["probe_c"], what=f"{tag} probe_c")
        if O:
            w_head = oracle.linear(want["h_n"][-1], *linear_params(head))
            assert_close(res["out"][rd].float().cpu().numpy(), w_head, what=f"{tag} head")
        done += 1


def test_sliced_two_tile_handoff_repeated(gpu):
    """Regression: the sliced kernel's staging waves read the shared copy of the upstream hand-off
    count in their first input wait.  It was zeroed only after the kernel's first barrier, so a wave
    could read what an earlier workgroup had left in LDS, take unpublished steps of the previous
    layer's hand-off as published and compute a whole 16-row tile from them (about 0.5% of forwards
    at padded H 256 with two tiles per workgroup, seen in random sweeps).  Two such geometries,
    alternated 200 times each: every forward equals its geometry's first bitwise, and each first
    forward matches the oracle on sampled rows."""
    device = torch.device("cuda")
    cases = []
    for I, H, L, O, B, T in ((20, 200, 3, 5, 600, 12), (7, 230, 4, 0, 300, 9)):
        torch.manual_seed(7 * H + B)
        lstm = torch.nn.LSTM(I, H, L, batch_first=True)
        head = torch.nn.Linear(H, O) if O else None
        x = torch.randn(B, T, I, generator=torch.Generator().manual_seed(B))
        params = [[getattr(lstm, f"{n}_l{l}").detach().cuda() for l in range(L)]
                  for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
        packed = gpu.pack(*params, head.weight.detach().cuda() if head else None,
                          head.bias.detach().cuda() if head else None)
        cases.append(((I, H, L, O), lstm, x, x.to(device, torch.float16), packed))

    def run(c):
        dims, _, _, xd, packed = c
        return gpu.forward(packed, dims, xd, want_out=dims[3] > 0, want_seq=True, want_state=True,
                           check_status=True)["out_seq"]

    firsts = [run(c).clone() for c in cases]
    for c, first in zip(cases, firsts):
        dims, lstm, x, _, _ = c
        rows = np.unique(np.r_[0:4, np.linspace(4, x.shape[0] - 1, 28).astype(int)])
        want = oracle.lstm_forward(x.numpy()[rows], oracle_layers(lstm), want_seq=True)["out_seq"]
        assert_close(first[torch.from_numpy(rows).to(device)].float().cpu().numpy(), want,
                     what=f"H={dims[1]} first forward vs oracle")
    _say("sliced two-tile hand-off: 400 alternating forwards")
    bad = []
    for it in range(200):
        for k, c in enumerate(cases):
            if not torch.equal(run(c), firsts[k]):
                bad.append((it, k))
    assert not bad, f"{len(bad)} forwards differ from their geometry's first: {bad[:10]}"
