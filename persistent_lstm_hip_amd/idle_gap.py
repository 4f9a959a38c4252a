"""Forward latency after an idle gap: how the GPU's clock management shapes back-to-back timings.

    python -m persistent_lstm_hip_amd.idle_gap [--hidden 128] [--layers 4] [--batch 512] [--seq 1000]

Runs the fp16 forward back to back with one event pair per forward: first from a fresh process, then
after idle gaps of 0 to 100 ms inserted into an otherwise continuous stream of forwards, and prints
the mean latency over forward windows after each gap.  On MI355X the shader clock falls within a few
forwards of any idle period (even one of a millisecond: the host synchronising between two phases of
a benchmark) and climbs back over ~40 ms of continuous work, so a protocol that times few forwards
right after a synchronisation measures part of that climb.  A diagnostic of the machine, not of the
kernels: every forward computes the same thing.
"""
from __future__ import annotations

import argparse
import statistics
import time

import torch


def _windows(t, bounds):
    return " ".join(f"[{i}:{j}] {statistics.mean(t[i:j]):.3f}" for i, j in bounds if j <= len(t))


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--input", type=int, default=5)
    ap.add_argument("--hidden", type=int, default=128)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--output", type=int, default=24)
    ap.add_argument("--batch", type=int, default=512)
    ap.add_argument("--seq", type=int, default=1000)
    args = ap.parse_args()
    if not torch.cuda.is_available():
        print("idle_gap: no HIP GPU visible")
        return 1
    from persistent_lstm_hip_amd import PersistentLSTMRegressor, StandardLSTMRegressor

    torch.manual_seed(42)
    native = StandardLSTMRegressor(args.input, args.hidden, args.output, args.layers).eval()
    model = PersistentLSTMRegressor.from_native_module(native).to("cuda").half().eval()
    x = torch.randn(args.batch, args.seq, args.input, generator=torch.Generator().manual_seed(1))
    x = x.to("cuda", torch.float16)

    def run(n):
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        with torch.inference_mode():
            for a, b in ev:
                a.record()
                model(x)
                b.record()
        torch.cuda.synchronize()
        return [a.elapsed_time(b) for a, b in ev]

    t = run(200)
    print("ms per forward, fresh process (the first includes the weights' packing):",
          _windows(t, [(1, 5), (5, 10), (10, 20), (20, 30), (30, 50), (50, 100), (100, 200)]), flush=True)
    for gap_ms in (0.0, 0.2, 1.0, 3.0, 10.0, 30.0, 100.0):
        run(100)
        if gap_ms:
            time.sleep(gap_ms / 1e3)
        t = run(40)
        print(f"after a {gap_ms:5.1f} ms idle gap:", _windows(t, [(0, 5), (5, 10), (10, 20), (20, 40)]), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
