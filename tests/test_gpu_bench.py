"""The benchmark's own lines run end to end on the GPU and print one JSON
line each: the encode workload (vectors/s with its MFMA roofline) and the
1,024-token decode workload (decode tokens/s with its HBM roofline)."""

import json

import pytest

pytestmark = pytest.mark.gpu


def _line(capsys):
    out = capsys.readouterr().out.strip().splitlines()
    return json.loads(out[-1])


def test_bench_encode_line(device, capsys):
    import bench

    assert bench.main(["--workload", "encode_4k", "--steps", "1", "--warmup", "0", "--no-cpu"]) == 0
    r = _line(capsys)
    assert r["unit"] == "vectors/s" and r["value"] > 0
    assert r["roofline"]["bound"] == "mfma" and 0 < r["roofline"]["frac"] < 1
    assert r["config"]["vectors_per_step"] == 2 * 4096 * 8
    assert r["warmup_run"]["ms"] >= r["warmup_run"]["floor_ms"]


def test_bench_decode_line(device, capsys):
    import bench

    assert bench.main(["--workload", "smoke_1k", "--steps", "5", "--warmup", "1", "--no-cpu"]) == 0
    r = _line(capsys)
    assert r["unit"] == "decode tokens/s" and r["value"] > 0 and r["steps"] == 5
    assert r["roofline"]["bound"] == "hbm" and r["bytes_per_step"] > 0
    assert r["warmup_run"]["steps_run"] >= 1
