"""Generate the golden fixtures in this directory with torch's fp32 CPU nn.LSTM / nn.Linear.

The reference repository ships no golden vectors, known-answer tests or fixtures for this path
(its only tests cover a scheduler heuristic), so these vectors come from torch's library LSTM, the
routine the reference's own CPU path restates (persistent_lstm_reference.cpp:7-64).  Weights are
rounded to fp16 before use so the fixtures store them losslessly as float16 and the GPU path runs on
exactly the same values.

    python tests/golden/make_golden.py     # rewrites c1.npz, c2_slice.npz, ragged_mini.npz
"""
from __future__ import annotations

import hashlib
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def seeded_modules(I, H, L, O, seed=42):
    torch.manual_seed(seed)
    lstm = torch.nn.LSTM(I, H, L, batch_first=True, dropout=0.2 if L > 1 else 0.0)
    lin = torch.nn.Linear(H, O)
    with torch.no_grad():  # make every parameter exactly representable in fp16
        for p in list(lstm.parameters()) + list(lin.parameters()):
            p.copy_(p.half().float())
    return lstm.eval(), lin.eval()


def weights_digest(lstm, lin) -> str:
    h = hashlib.sha256()
    for p in list(lstm.parameters()) + list(lin.parameters()):
        h.update(p.detach().half().numpy().tobytes())
    return h.hexdigest()


def states_after(lstm, x, steps, lengths=None):
    hs, cs = [], []
    with torch.inference_mode():
        for t in steps:
            if lengths is None:
                _, (h, c) = lstm(x[:, :t])
            else:
                lt = torch.clamp(lengths, max=t)
                keep = lt > 0
                packed = torch.nn.utils.rnn.pack_padded_sequence(x[keep, :t], lt[keep], batch_first=True,
                                                                 enforce_sorted=False)
                _, (hk, ck) = lstm(packed)
                h = torch.zeros(lstm.num_layers, x.shape[0], lstm.hidden_size)
                c = torch.zeros_like(h)
                h[:, keep], c[:, keep] = hk, ck
            hs.append(h.numpy())
            cs.append(c.numpy())
    return np.stack(hs), np.stack(cs)


def layer_arrays(lstm):
    d = {}
    for l in range(lstm.num_layers):
        for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
            d[f"{n}_l{l}"] = getattr(lstm, f"{n}_l{l}").detach().half().numpy()
    return d


def make_c1():
    """Config 1: 1 layer, I=5, H=128, O=24, B=8, T=64."""
    I, H, L, O, B, T = 5, 128, 1, 24, 8, 64
    lstm, lin = seeded_modules(I, H, L, O)
    x = torch.randn(B, T, I, generator=torch.Generator().manual_seed(1)).half().float()
    with torch.inference_mode():
        seq, _ = lstm(x)
        out = lin(seq[:, -1])
    steps = (1, 32, 64)
    hs, cs = states_after(lstm, x, steps)
    np.savez_compressed(os.path.join(HERE, "c1.npz"), x=x.half().numpy(), out=out.numpy(),
                        probe_steps=np.array(steps), probe_h=hs, probe_c=cs,
                        linear_weight=lin.weight.detach().half().numpy(), linear_bias=lin.bias.detach().half().numpy(),
                        dims=np.array([I, H, L, O]), **layer_arrays(lstm))


def make_c2_slice():
    """Config 2 (I=5, H=128, L=4, O=24, T=1000), 8 batch rows.  Weights are regenerated from the
    seed by the test (their fp16 digest is stored to detect RNG drift); x and expected values are
    stored."""
    I, H, L, O, B, T = 5, 128, 4, 24, 8, 1000
    lstm, lin = seeded_modules(I, H, L, O)
    x = torch.randn(512, T, I, generator=torch.Generator().manual_seed(1))[:B].half().float()
    with torch.inference_mode():
        seq, _ = lstm(x)
        out = lin(seq[:, -1])
    steps = (1, 100, 1000)
    hs, cs = states_after(lstm, x, steps)
    np.savez_compressed(os.path.join(HERE, "c2_slice.npz"), x=x.half().numpy(), out=out.numpy(),
                        probe_steps=np.array(steps), probe_h=hs.astype(np.float32), probe_c=cs.astype(np.float32),
                        dims=np.array([I, H, L, O]), weights_sha256=np.array(weights_digest(lstm, lin)))


def make_ragged_mini():
    """Packed-sequence semantics: I=5, H=32, L=2, O=3, B=8, T=64, lengths sorted descending."""
    I, H, L, O, B, T = 5, 32, 2, 3, 8, 64
    lstm, lin = seeded_modules(I, H, L, O)
    x = torch.randn(B, T, I, generator=torch.Generator().manual_seed(1)).half().float()
    lengths = torch.sort(torch.randint(1, T + 1, (B,), generator=torch.Generator().manual_seed(2)),
                         descending=True).values
    packed = torch.nn.utils.rnn.pack_padded_sequence(x, lengths, batch_first=True)
    with torch.inference_mode():
        seq_p, (h, c) = lstm(packed)
        seq, _ = torch.nn.utils.rnn.pad_packed_sequence(seq_p, batch_first=True, total_length=T)
        out = lin(h[-1])
    steps = (1, 32, 64)
    hs, cs = states_after(lstm, x, steps, lengths)
    np.savez_compressed(os.path.join(HERE, "ragged_mini.npz"), x=x.half().numpy(), lengths=lengths.numpy(),
                        out=out.numpy(), out_seq=seq.numpy(), h_n=h.numpy(), c_n=c.numpy(),
                        probe_steps=np.array(steps), probe_h=hs, probe_c=cs,
                        linear_weight=lin.weight.detach().half().numpy(), linear_bias=lin.bias.detach().half().numpy(),
                        dims=np.array([I, H, L, O]), **layer_arrays(lstm))


if __name__ == "__main__":
    make_c1()
    make_c2_slice()
    make_ragged_mini()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
