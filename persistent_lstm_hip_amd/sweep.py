"""Shape-sweep timing and comparison in the reference's CSV formats.

    python -m persistent_lstm_hip_amd.sweep run [--backend hip|native] [--cases 128:512,256:512,512:128]
                                                [--iters 100] [--warmup 10] [--input randn|ones]
    python -m persistent_lstm_hip_amd.sweep compare --native A.txt --adaptive B.txt

`run` times the 4-layer regressor (input 5, output 24 unless overridden) for each hidden:batch[:seq]
case as the reference's run_native_lstm_sweep.py does (persistent_lstm_hip/run_native_lstm_sweep.py:
63-119): `warmup` untimed forwards, then `iters` forwards between two device synchronisations on the
wall clock; throughput = iters / elapsed * batch samples/s; per case the median over `repeats`.  It
prints the per-case lines and the summary block

    hidden,batch,seq,elapsed_s,throughput,kernel

(run_native_lstm_sweep.py:116-119).  `--backend hip` runs this build (kernel column: its backend
name), `--backend native` torch's nn.LSTM (kernel column: native_pytorch_lstm).  The reference feeds
torch.ones, which this build's uniform-batch shortcut answers with one row; the default input here
is therefore randn (seeded), and `--input ones` reproduces the reference's protocol.  The
reference's environment variables (NATIVE_LSTM_SWEEP, MIOPEN_ADAPTIVE_INPUT/OUTPUT/LAYERS/ITERS/SEQ,
NATIVE_LSTM_WARMUP, NATIVE_LSTM_SWEEP_REPEATS, NATIVE_LSTM_DEVICE) give the defaults.

`compare` joins two sweep outputs on (hidden, batch, seq) and prints compare_lstm_sweeps.py's
columns (compare_lstm_sweeps.py:46-87):

    hidden,batch,seq,native_elapsed,adaptive_elapsed,elapsed_speedup,native_tput,adaptive_tput,tput_speedup,kernel
"""
from __future__ import annotations

import argparse
import csv
import os
import sys
import time
from dataclasses import dataclass
from io import StringIO
from statistics import median
from typing import Dict, List, Sequence, Tuple

SUMMARY_HEADER = "hidden,batch,seq,elapsed_s,throughput,kernel"
COMPARE_HEADER = ("hidden,batch,seq,native_elapsed,adaptive_elapsed,elapsed_speedup,native_tput,adaptive_tput,"
                  "tput_speedup,kernel")
NATIVE_KERNEL = "native_pytorch_lstm"


@dataclass(frozen=True)
class ShapeCase:
    hidden: int
    batch: int
    seq: int


@dataclass(frozen=True)
class SweepRow:
    hidden: int
    batch: int
    seq: int
    elapsed_s: float
    throughput: float
    kernel: str


def parse_cases(raw: str, default_seq: int) -> List[ShapeCase]:
    """'128:512,256:512:300' -> cases; a missing seq is default_seq (run_native_lstm_sweep.py:35-52)."""
    cases: List[ShapeCase] = []
    for piece in raw.split(","):
        piece = piece.strip()
        if not piece:
            continue
        parts = piece.split(":")
        if len(parts) not in (2, 3):
            raise ValueError("cases must look like 128:512,256:512,512:128 or hidden:batch:seq")
        hidden, batch = int(parts[0]), int(parts[1])
        seq = int(parts[2]) if len(parts) == 3 else default_seq
        if hidden <= 0 or batch <= 0 or seq <= 0:
            raise ValueError(f"case {piece!r}: hidden, batch and seq must be positive")
        cases.append(ShapeCase(hidden, batch, seq))
    if not cases:
        raise ValueError("no sweep cases given")
    return cases


def format_summary(rows: Sequence[SweepRow]) -> str:
    lines = [SUMMARY_HEADER]
    for r in rows:
        lines.append(f"{r.hidden},{r.batch},{r.seq},{r.elapsed_s:.6f},{r.throughput:.3f},{r.kernel}")
    return "\n".join(lines)


def extract_csv_block(text: str) -> str:
    """The last summary block of a sweep output (compare_lstm_sweeps.py:28-43)."""
    lines = text.splitlines()
    header_idx = -1
    for idx, line in enumerate(lines):
        if line.strip().startswith("hidden,batch,seq,elapsed_s,throughput"):
            header_idx = idx
    if header_idx < 0:
        raise ValueError("could not find sweep summary CSV header")
    block: List[str] = []
    for line in lines[header_idx:]:
        stripped = line.strip()
        if not stripped:
            break
        if stripped.startswith("hidden,") or stripped[0].isdigit():
            block.append(stripped)
    return "\n".join(block)


def parse_rows(text: str) -> Dict[Tuple[int, int, int], SweepRow]:
    rows: Dict[Tuple[int, int, int], SweepRow] = {}
    for raw in csv.DictReader(StringIO(extract_csv_block(text))):
        key = (int(raw["hidden"]), int(raw["batch"]), int(raw["seq"]))
        rows[key] = SweepRow(*key, elapsed_s=float(raw["elapsed_s"]), throughput=float(raw["throughput"]),
                             kernel=raw.get("kernel") or "")
    return rows


def compare(native_text: str, adaptive_text: str) -> str:
    """Joined rows of two sweep outputs (compare_lstm_sweeps.py:64-87): elapsed speedup = native /
    other elapsed, throughput speedup = other / native throughput, kernel of the other sweep."""
    native, other = parse_rows(native_text), parse_rows(adaptive_text)
    common = sorted(set(native) & set(other))
    if not common:
        raise ValueError("no common hidden,batch,seq rows found")
    lines = [COMPARE_HEADER]
    for key in common:
        n, a = native[key], other[key]
        lines.append(f"{a.hidden},{a.batch},{a.seq},{n.elapsed_s:.6f},{a.elapsed_s:.6f},{n.elapsed_s / a.elapsed_s:.3f},"
                     f"{n.throughput:.3f},{a.throughput:.3f},{a.throughput / n.throughput:.3f},{a.kernel}")
    return "\n".join(lines)


def _env_int(name: str, default: int) -> int:
    return int(os.environ.get(name, str(default)))


def run(cases: Sequence[ShapeCase], *, backend: str = "hip", input_size: int = 5, output_size: int = 24,
        num_layers: int = 4, iters: int = 100, warmup: int = 10, repeats: int = 1, input_kind: str = "randn",
        device: str = "cuda:0", out=sys.stdout) -> List[SweepRow]:
    """Time every case; prints the reference's per-case lines to `out` and returns the summary rows."""
    import torch

    from .model import PersistentLSTMRegressor, StandardLSTMRegressor

    if backend not in ("hip", "native"):
        raise ValueError("backend must be 'hip' or 'native'")
    if input_kind not in ("randn", "ones"):
        raise ValueError("input must be 'randn' or 'ones'")
    if iters <= 0 or warmup < 0 or repeats <= 0:
        raise ValueError("iters and repeats must be positive, warmup non-negative")
    rows: List[SweepRow] = []
    for case in cases:
        elapsed_values, tput_values = [], []
        kernel = NATIVE_KERNEL
        for rep in range(repeats):
            label = f" repeat={rep + 1}/{repeats}" if repeats > 1 else ""
            print(f"\n=== {backend} hidden={case.hidden} batch={case.batch} seq={case.seq}{label} ===", file=out,
                  flush=True)
            torch.manual_seed(42)
            native = StandardLSTMRegressor(input_size, case.hidden, output_size, num_layers).eval()
            if backend == "hip":
                model = PersistentLSTMRegressor.from_native_module(native).to(device).half().eval()
                kernel = model.backend_name
            else:
                model = native.to(device).half().eval()
            shape = (case.batch, case.seq, input_size)
            if input_kind == "ones":
                x = torch.ones(shape, device=device, dtype=torch.float16)
            else:
                x = torch.randn(shape, generator=torch.Generator().manual_seed(1)).to(device, torch.float16)
            with torch.inference_mode():
                for _ in range(warmup):
                    model(x)
                torch.cuda.synchronize(device)
                start = time.time()
                for _ in range(iters):
                    model(x)
                torch.cuda.synchronize(device)
            elapsed = time.time() - start
            tput = iters / elapsed * case.batch
            print(f"backend: {kernel}", file=out)
            print(f"elapsed={elapsed:.6f}s", file=out)
            print(f"throughput={tput:.3f} samples/s", file=out, flush=True)
            elapsed_values.append(elapsed)
            tput_values.append(tput)
        rows.append(SweepRow(case.hidden, case.batch, case.seq, median(elapsed_values), median(tput_values), kernel))
    print("\nsummary:", file=out)
    print(format_summary(rows), file=out, flush=True)
    return rows


def _read(path: str) -> str:
    if path == "-":
        return sys.stdin.read()
    with open(path, encoding="utf-8") as f:
        return f.read()


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="LSTM shape sweeps in the reference's CSV formats")
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run", help="time hidden:batch[:seq] cases")
    r.add_argument("--backend", default="hip", choices=("hip", "native"))
    r.add_argument("--cases", default=os.environ.get("NATIVE_LSTM_SWEEP",
                                                     os.environ.get("MIOPEN_ADAPTIVE_SWEEP", "128:512,256:512,512:128")))
    r.add_argument("--seq", type=int, default=_env_int("MIOPEN_ADAPTIVE_SEQ", 1000))
    r.add_argument("--input-size", type=int, default=_env_int("MIOPEN_ADAPTIVE_INPUT", 5))
    r.add_argument("--output-size", type=int, default=_env_int("MIOPEN_ADAPTIVE_OUTPUT", 24))
    r.add_argument("--layers", type=int, default=_env_int("MIOPEN_ADAPTIVE_LAYERS", 4))
    r.add_argument("--iters", type=int, default=_env_int("MIOPEN_ADAPTIVE_ITERS", 100))
    r.add_argument("--warmup", type=int, default=_env_int("NATIVE_LSTM_WARMUP", 10))
    r.add_argument("--repeats", type=int, default=_env_int("NATIVE_LSTM_SWEEP_REPEATS", 1))
    r.add_argument("--input", default="randn", choices=("randn", "ones"))
    r.add_argument("--device", default=os.environ.get("NATIVE_LSTM_DEVICE", "cuda:0"))
    c = sub.add_parser("compare", help="join two sweep outputs")
    c.add_argument("--native", required=True, help="native sweep output, or '-' for stdin")
    c.add_argument("--adaptive", required=True, help="the other sweep output, or '-' for stdin")
    args = ap.parse_args(argv)
    if args.cmd == "compare":
        print(compare(_read(args.native), _read(args.adaptive)))
        return 0
    run(parse_cases(args.cases, args.seq), backend=args.backend, input_size=args.input_size,
        output_size=args.output_size, num_layers=args.layers, iters=args.iters, warmup=args.warmup,
        repeats=args.repeats, input_kind=args.input, device=args.device)
    return 0


if __name__ == "__main__":
    sys.exit(main())
