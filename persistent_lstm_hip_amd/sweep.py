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
import os
import re
import sys
import time
from statistics import median
from typing import Dict, Iterable, List, NamedTuple, Sequence, Tuple

SUMMARY_HEADER = "hidden,batch,seq,elapsed_s,throughput,kernel"
COMPARE_HEADER = ("hidden,batch,seq,native_elapsed,adaptive_elapsed,elapsed_speedup,native_tput,adaptive_tput,"
                  "tput_speedup,kernel")
NATIVE_KERNEL = "native_pytorch_lstm"

Shape = Tuple[int, int, int]  # (hidden, batch, seq): the key that joins two sweeps


class ShapeCase(NamedTuple):
    hidden: int
    batch: int
    seq: int


class SweepRow(NamedTuple):
    hidden: int
    batch: int
    seq: int
    elapsed_s: float
    throughput: float
    kernel: str

    @property
    def shape(self) -> Shape:
        return (self.hidden, self.batch, self.seq)

    def csv(self) -> str:
        return f"{self.hidden},{self.batch},{self.seq},{self.elapsed_s:.6f},{self.throughput:.3f},{self.kernel}"


# "hidden:batch" or "hidden:batch:seq", decimal integers, blanks around the item allowed.
_CASE = re.compile(r"\s*(\d+):(\d+)(?::(\d+))?\s*")
# One summary record: three integers, two numbers and the (possibly empty) kernel name.
_RECORD = re.compile(r"(\d+),(\d+),(\d+),([-+.\deE]+|nan|inf),([-+.\deE]+|nan|inf),([^,]*)")


def parse_cases(raw: str, default_seq: int) -> List[ShapeCase]:
    """'128:512,256:512:300' -> cases (the sweep's case syntax, run_native_lstm_sweep.py:35-52); a
    missing seq is default_seq; empty items are skipped."""
    items = [item for item in raw.split(",") if item.strip()]
    if not items:
        raise ValueError("no sweep cases given")
    cases = []
    for item in items:
        m = _CASE.fullmatch(item)
        if m is None:
            raise ValueError(f"case {item.strip()!r}: expected hidden:batch or hidden:batch:seq "
                             "(e.g. 128:512,256:512,512:128)")
        case = ShapeCase(int(m[1]), int(m[2]), int(m[3]) if m[3] is not None else default_seq)
        if min(case) <= 0:
            raise ValueError(f"case {item.strip()!r}: hidden, batch and seq must be positive")
        cases.append(case)
    return cases


def format_summary(rows: Iterable[SweepRow]) -> str:
    return "\n".join([SUMMARY_HEADER] + [r.csv() for r in rows])


def read_summary(text: str) -> Dict[Shape, SweepRow]:
    """The rows of the last summary block of a sweep output (the block starts at a line holding the
    summary header and runs over the record lines right after it), keyed by shape; a later row of
    one shape replaces an earlier one.  ValueError if the text holds no header."""
    lines = [line.strip() for line in text.splitlines()]
    starts = [i for i, line in enumerate(lines) if line.startswith(SUMMARY_HEADER.rsplit(",", 1)[0])]
    if not starts:
        raise ValueError("no sweep summary block (header 'hidden,batch,seq,elapsed_s,throughput,...') found")
    table: Dict[Shape, SweepRow] = {}
    for line in lines[starts[-1] + 1:]:
        m = _RECORD.fullmatch(line)
        if m is None:
            break
        row = SweepRow(int(m[1]), int(m[2]), int(m[3]), float(m[4]), float(m[5]), m[6])
        table[row.shape] = row
    return table


# A summary of this build may be compared as either side; the joined line's kernel column names the
# second ("adaptive") sweep's kernel, as compare_lstm_sweeps.py:77-87 prints it.
def join_sweeps(base: Dict[Shape, SweepRow], other: Dict[Shape, SweepRow]) -> List[Tuple[SweepRow, SweepRow]]:
    """(base row, other row) for every shape both sweeps measured, in shape order."""
    return [(base[k], other[k]) for k in sorted(base.keys() & other.keys())]


def compare(native_text: str, adaptive_text: str) -> str:
    """compare_lstm_sweeps.py's joined table of two sweep outputs: elapsed speedup = base elapsed /
    other elapsed, throughput speedup = other / base throughput."""
    pairs = join_sweeps(read_summary(native_text), read_summary(adaptive_text))
    if not pairs:
        raise ValueError("no common hidden,batch,seq rows found")
    out = [COMPARE_HEADER]
    for base, other in pairs:
        fields = [str(v) for v in other.shape]
        fields += [f"{base.elapsed_s:.6f}", f"{other.elapsed_s:.6f}", f"{base.elapsed_s / other.elapsed_s:.3f}"]
        fields += [f"{base.throughput:.3f}", f"{other.throughput:.3f}", f"{other.throughput / base.throughput:.3f}"]
        out.append(",".join(fields + [other.kernel]))
    return "\n".join(out)


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
