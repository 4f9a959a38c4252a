"""The sweep harness's formats (CPU): the reference's summary CSV
(run_native_lstm_sweep.py:116-119) and its joiner's columns (compare_lstm_sweeps.py:77-87)."""
from __future__ import annotations

import io

import pytest
import torch

from persistent_lstm_hip_amd import sweep

NATIVE_OUT = """
=== native hidden=128 batch=512 seq=1000 ===
backend: native_pytorch_lstm
elapsed=8.210000s
throughput=6236.297 samples/s

summary:
hidden,batch,seq,elapsed_s,throughput,kernel
128,512,1000,8.210000,6236.297,native_pytorch_lstm
256,512,1000,11.770000,4350.042,native_pytorch_lstm
512,128,1000,5.000000,2560.000,native_pytorch_lstm
"""

HIP_OUT = """summary:
hidden,batch,seq,elapsed_s,throughput,kernel
128,512,1000,0.100000,512000.000,hip_mi355x_persistent_wavefront
512,128,1000,0.500000,25600.000,hip_mi355x_persistent_wavefront
64,32,100,0.010000,320000.000,hip_mi355x_persistent_wavefront
"""


def test_parse_cases():
    cases = sweep.parse_cases("128:512, 256:512:300,", default_seq=1000)
    assert cases == [sweep.ShapeCase(128, 512, 1000), sweep.ShapeCase(256, 512, 300)]
    for bad in ("128", "128:512:1:2", "", "0:5"):
        with pytest.raises(ValueError):
            sweep.parse_cases(bad, 1000)


def test_summary_round_trip():
    rows = [sweep.SweepRow(128, 512, 1000, 0.0881234567, 581034.4567, "k1"),
            sweep.SweepRow(512, 64, 50, 1.5, 4266.6666, "k2")]
    text = "noise\n" + sweep.format_summary(rows) + "\n\ntrailing"
    assert text.splitlines()[1] == sweep.SUMMARY_HEADER
    back = sweep.parse_rows(text)
    assert back[(128, 512, 1000)] == sweep.SweepRow(128, 512, 1000, 0.088123, 581034.457, "k1")
    assert back[(512, 64, 50)].kernel == "k2"


def test_extract_uses_the_last_summary_block():
    text = NATIVE_OUT + "\nsummary:\n" + sweep.SUMMARY_HEADER + "\n64,8,10,1.000000,80.000,late\n"
    assert set(sweep.parse_rows(text)) == {(64, 8, 10)}
    with pytest.raises(ValueError):
        sweep.parse_rows("no csv here")


def test_compare_joins_common_rows():
    out = sweep.compare(NATIVE_OUT, HIP_OUT).splitlines()
    assert out[0] == sweep.COMPARE_HEADER
    assert out[1:] == [
        "128,512,1000,8.210000,0.100000,82.100,6236.297,512000.000,82.100,hip_mi355x_persistent_wavefront",
        "512,128,1000,5.000000,0.500000,10.000,2560.000,25600.000,10.000,hip_mi355x_persistent_wavefront",
    ]
    with pytest.raises(ValueError, match="no common"):
        sweep.compare(NATIVE_OUT, "hidden,batch,seq,elapsed_s,throughput,kernel\n1,1,1,1.0,1.0,x\n")


def test_cli_compare(tmp_path, capsys):
    a, b = tmp_path / "n.txt", tmp_path / "h.txt"
    a.write_text(NATIVE_OUT)
    b.write_text(HIP_OUT)
    assert sweep.main(["compare", "--native", str(a), "--adaptive", str(b)]) == 0
    assert capsys.readouterr().out.splitlines()[0] == sweep.COMPARE_HEADER


def test_run_validates_arguments():
    with pytest.raises(ValueError):
        sweep.run([sweep.ShapeCase(8, 2, 3)], backend="cpu")
    with pytest.raises(ValueError):
        sweep.run([sweep.ShapeCase(8, 2, 3)], iters=0)


@pytest.mark.gpu
def test_run_hip_prints_a_parsable_summary():
    buf = io.StringIO()
    rows = sweep.run([sweep.ShapeCase(64, 16, 20), sweep.ShapeCase(200, 8, 10)], iters=3, warmup=1, out=buf)
    assert [(r.hidden, r.batch, r.seq) for r in rows] == [(64, 16, 20), (200, 8, 10)]
    parsed = sweep.parse_rows(buf.getvalue())
    assert parsed[(64, 16, 20)].kernel == "hip_mi355x_persistent_wavefront" and parsed[(64, 16, 20)].throughput > 0
    assert torch.cuda.is_available()
