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
    assert sweep.parse_cases(" 64:8 ", default_seq=7) == [sweep.ShapeCase(64, 8, 7)]
    for bad in ("128", "128:512:1:2", "", "0:5", "a:b", "12:-3", ",,"):
        with pytest.raises(ValueError):
            sweep.parse_cases(bad, 1000)


def test_summary_round_trip():
    rows = [sweep.SweepRow(128, 512, 1000, 0.0881234567, 581034.4567, "k1"),
            sweep.SweepRow(512, 64, 50, 1.5, 4266.6666, "k2")]
    text = "noise\n" + sweep.format_summary(rows) + "\n\ntrailing"
    assert text.splitlines()[1] == sweep.SUMMARY_HEADER
    back = sweep.read_summary(text)
    assert back[(128, 512, 1000)] == sweep.SweepRow(128, 512, 1000, 0.088123, 581034.457, "k1")
    assert back[(512, 64, 50)].kernel == "k2"


def test_extract_uses_the_last_summary_block():
    text = NATIVE_OUT + "\nsummary:\n" + sweep.SUMMARY_HEADER + "\n64,8,10,1.000000,80.000,late\n"
    assert set(sweep.read_summary(text)) == {(64, 8, 10)}
    with pytest.raises(ValueError):
        sweep.read_summary("no csv here")


def test_summary_block_ends_at_the_first_non_record_line():
    text = (sweep.SUMMARY_HEADER + "\n  128,512,1000,1.5,2.5,k  \n256,8,10,1e-3,4E+2,\nnot a record\n"
            "512,1,1,1.0,1.0,after\n")
    rows = sweep.read_summary(text)
    assert set(rows) == {(128, 512, 1000), (256, 8, 10)}
    assert rows[(256, 8, 10)] == sweep.SweepRow(256, 8, 10, 1e-3, 400.0, "")
    # a header with nothing after it is an empty table, and a repeated shape keeps its last row
    assert sweep.read_summary("x\n" + sweep.SUMMARY_HEADER) == {}
    dup = sweep.SUMMARY_HEADER + "\n1,2,3,1.0,1.0,a\n1,2,3,2.0,2.0,b\n"
    assert sweep.read_summary(dup)[(1, 2, 3)].kernel == "b"


def test_join_sweeps_in_shape_order():
    a = sweep.read_summary(NATIVE_OUT)
    b = sweep.read_summary(HIP_OUT)
    pairs = sweep.join_sweeps(a, b)
    assert [p[0].shape for p in pairs] == [(128, 512, 1000), (512, 128, 1000)]
    assert all(x.shape == y.shape for x, y in pairs)
    assert sweep.join_sweeps(a, {}) == []


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
    parsed = sweep.read_summary(buf.getvalue())
    assert parsed[(64, 16, 20)].kernel == "hip_mi355x_persistent_wavefront" and parsed[(64, 16, 20)].throughput > 0
    assert torch.cuda.is_available()
